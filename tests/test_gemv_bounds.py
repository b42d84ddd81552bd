"""Device-free: every weight load of the GEMV kernels stays inside the weight image or the
sink, at every config shape and column count that runs on the GEMV.

The library replays a launch's loads on the host (qmm_internal_gemv_extent, declared in
arcint_amd/csrc/qmm_internal.h): it plans the launch as qmm_mul_mat / qmm_mul_mat_id do and
walks every work-group, wave and stage with the kernels' own index functions, including the
one stage per wave that the MFMA kernel's register ring loads past its last one (from the
sink; the v_dot4 kernels load none).  Checked here: no load outside [0, image bytes) of the
matrices it may address, none past the sink, every (task, tile, group) of the product loaded
exactly once (the plan covers K and the rows with no gap or overlap), and at most one sink
load per wave that streams anything."""
import ctypes as C

import numpy as np
import pytest

from arcint_amd import qmm

SINK_BYTES = 32768


def extent(qtype, ne0, N, nbatch=1, n_used=0):
    L = qmm.load()
    f = L.qmm_internal_gemv_extent
    f.argtypes = [C.c_int32, C.POINTER(C.c_int64), C.c_int64, C.c_int64, C.c_int64, C.POINTER(C.c_int64)]
    out = (C.c_int64 * 8)()
    ne = (C.c_int64 * 4)(*qmm._ne4(ne0))
    rc = f(qtype, ne, N, nbatch, n_used, out)
    if rc == 2:                                                    # QMM_ERR_UNSUPPORTED: runs on the GEMM
        return None
    assert rc == 0, rc
    keys = ("image_bytes", "real_lo", "real_hi", "sink_hi", "real_loads", "sink_loads", "bad", "read_end")
    return dict(zip(keys, list(out)))


def tiles_groups(ne0):
    M, K = ne0[1], ne0[0]
    return (M + 63) // 64, (K + 255) // 256


SHAPES = [  # (type, M, K): the configs' matrices, the adjacent types on them, ragged shapes
    (qmm.Q4_0, 4096, 4096), (qmm.Q4_0, 11008, 4096), (qmm.Q4_0, 4096, 11008),
    (qmm.Q4_K, 17408, 5120), (qmm.Q6_K, 5120, 17408), (qmm.Q6_K, 151936, 5120),
    (qmm.Q4_K, 12288, 5120), (qmm.Q4_K, 1024, 5120), (qmm.Q4_K, 5120, 6144),
    (qmm.IQ4_XS, 14336, 4096), (qmm.IQ4_XS, 4096, 14336), (qmm.Q8_0, 14336, 4096), (qmm.Q8_0, 4096, 14336),
    (qmm.Q5_K, 17408, 5120), (qmm.IQ4_NL, 14336, 4096),
    (qmm.Q4_0, 300, 640), (qmm.Q8_0, 129, 416), (qmm.Q6_K, 70, 768), (qmm.IQ4_XS, 1, 256), (qmm.Q4_K, 65, 256),
]
COLS = [1, 2, 3, 4, 5, 8, 9, 12, 16, 17, 24, 32, 33, 40, 64, 96, 100, 127]


def check(e, tasks_times_tiles_groups=None):
    assert e["bad"] == 0, e
    assert 0 <= e["real_lo"] and e["real_hi"] <= e["image_bytes"], e
    assert e["sink_hi"] <= SINK_BYTES, e
    assert e["real_loads"] >= 1 and e["real_loads"] >= e["sink_loads"], e
    if tasks_times_tiles_groups:
        nst, r = divmod(e["real_loads"], tasks_times_tiles_groups)
        assert r == 0 and nst in (1, 2), (e, tasks_times_tiles_groups)


@pytest.mark.parametrize("qtype,M,K", SHAPES)
def test_gemv_loads_in_bounds(qtype, M, K):
    ran = 0
    for N in COLS:
        ne0 = (K, M)
        e = extent(qtype, ne0, N)
        if e is None:
            continue
        fake = qmm.Buffer(ptr=0x1000, size=1 << 44)
        info = qmm.describe_mul_mat(qmm.Tensor(fake, qtype, ne0), qmm.Tensor(fake, qmm.F32, (K, N)),
                                    qmm.Tensor(fake, qmm.F32, (M, N)))
        nt, G = tiles_groups(ne0)
        check(e, info["tasks"] * nt * G)
        ran += 1
    assert ran >= 1


@pytest.mark.parametrize("qtype", [qmm.Q4_K, qmm.Q4_0, qmm.Q6_K])
@pytest.mark.parametrize("N", [1, 4, 21])
def test_gemv_loads_broadcast(qtype, N):
    """two matrices broadcast over four batches: the last matrix's tiles end the image"""
    e = extent(qtype, (512, 80, 2), N, nbatch=4)
    nt, G = tiles_groups((512, 80))
    check(e)
    assert e["real_hi"] == e["image_bytes"]


@pytest.mark.parametrize("K,M,E,n_used", [(2048, 512, 512, 10), (512, 2048, 512, 10), (512, 96, 16, 4),
                                          (256, 64, 16, 4)])
@pytest.mark.parametrize("T", [1, 4, 19, 256, 1024])
def test_mul_mat_id_loads_in_bounds(K, M, E, n_used, T):
    """MUL_MAT_ID task lists (config 3's gate/up and down stacks): every task on the first and
    on the last expert stays inside the stack"""
    e = extent(qmm.Q4_K, (K, M, E), T, n_used=n_used)
    check(e)
    nt, G = tiles_groups((K, M))
    assert e["real_loads"] % (nt * G) == 0
    # the last expert's last tile-group ends the stack's image
    assert e["real_hi"] == e["image_bytes"]


def test_sink_covers_every_stage_extent():
    for qtype in qmm.QUANT_TYPES:
        e = extent(qtype, (256, 64), 1)
        assert e["read_end"] <= SINK_BYTES
        assert e["read_end"] * ((64 + 63) // 64) * 1 <= e["image_bytes"]


@pytest.mark.parametrize("qtype,M,K", SHAPES)
def test_fused_split_loads_in_bounds(monkeypatch, qtype, M, K):
    """the fused kernel with K split over work-groups (forced at every size, 1 and 4 waves a
    work-group): its loads stay inside the image and the sink, every tile-group once"""
    monkeypatch.setenv("QMM_GEMV_FQS", "1")
    fake = qmm.Buffer(ptr=0x1000, size=1 << 44)
    for W in ("1", "4"):
        monkeypatch.setenv("QMM_GEMV_FQS_W", W)
        for N in (1, 2):
            ne0 = (K, M)
            e = extent(qtype, ne0, N)
            info = qmm.describe_mul_mat(qmm.Tensor(fake, qtype, ne0), qmm.Tensor(fake, qmm.F32, (K, N)),
                                        qmm.Tensor(fake, qmm.F32, (M, N)))
            assert info["path"] == "gemv-fq", info
            nt, G = tiles_groups(ne0)
            check(e, info["tasks"] * nt * G)
            if G > int(W):
                assert info["k_slices"] == -(-G // int(W)) or info["k_slices"] == 1, info
