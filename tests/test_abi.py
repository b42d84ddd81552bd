"""The C ABI: libqmm.so loads, exports every function include/qmm.h declares,
and its host-only queries answer without a device.  CPU only."""
import ctypes as C
import os
import re

import pytest

from arcint_amd import qmm

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "qmm.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qmm_[a-z_0-9]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert header_functions() == sorted(qmm.EXPORTS)


def test_library_exports_every_declared_symbol():
    L = qmm.load()
    missing = [f for f in header_functions() if not hasattr(L, f)]
    assert not missing


def test_type_table():
    assert qmm.type_block(qmm.Q4_0) == (32, 18)
    assert qmm.type_block(qmm.Q8_0) == (32, 34)
    assert qmm.type_block(qmm.Q4_K) == (256, 144)
    assert qmm.type_block(qmm.Q6_K) == (256, 210)
    assert qmm.type_block(qmm.IQ4_XS) == (256, 136)
    assert qmm.type_block(qmm.F32) == (1, 4)
    with pytest.raises(qmm.QmmError):
        qmm.type_block(99)


def test_sizes():
    assert qmm.nbytes(qmm.Q4_K, (5120, 17408)) == 17408 * 20 * 144
    # planar layouts: every plane 256-byte aligned, never smaller than GGUF bytes
    for t in qmm.QUANT_TYPES:
        bl, bb = qmm.type_block(t)
        for rows in (1, 3, 1000):
            ne = (bl * 4, rows)
            assert qmm.alloc_size(t, ne) >= qmm.nbytes(t, ne)
            assert qmm.alloc_size(t, ne) % 256 == 0
    assert qmm.nbytes(qmm.Q4_0, (33, 1)) == 0          # not whole blocks


def test_supports_op_without_device():
    L = qmm.load()
    fake = qmm.Buffer(ptr=0x1000, size=1 << 40)

    def T(t, ne):
        return qmm.Tensor(fake, t, ne)

    w, x, y = T(qmm.Q4_K, (512, 64)), T(qmm.F32, (512, 3)), T(qmm.F32, (64, 3))
    buf = C.create_string_buffer(128)
    assert L.qmm_supports_op(None, qmm.OP_MUL_MAT, C.byref(w.c), C.byref(x.c), None, C.byref(y.c), buf, 128) == 1
    bad = T(qmm.F32, (64, 4))
    assert L.qmm_supports_op(None, qmm.OP_MUL_MAT, C.byref(w.c), C.byref(x.c), None, C.byref(bad.c), buf, 128) == 0
    assert b"dst shape" in buf.value
    w3 = T(qmm.Q4_K, (300, 64))                       # K not whole super-blocks
    assert L.qmm_supports_op(None, qmm.OP_MUL_MAT, C.byref(w3.c), C.byref(x.c), None, C.byref(y.c), buf, 128) == 0
    # MUL_MAT_ID shapes
    we = T(qmm.Q4_K, (512, 64, 8))
    xe = T(qmm.F32, (512, 1, 5))
    ids = T(qmm.I32, (2, 5))
    ye = T(qmm.F32, (64, 2, 5))
    assert L.qmm_supports_op(None, qmm.OP_MUL_MAT_ID, C.byref(we.c), C.byref(xe.c), C.byref(ids.c), C.byref(ye.c), buf, 128) == 1
    xe3 = T(qmm.F32, (512, 3, 5))                     # ne11 must be 1 or n_used
    assert L.qmm_supports_op(None, qmm.OP_MUL_MAT_ID, C.byref(we.c), C.byref(xe3.c), C.byref(ids.c), C.byref(ye.c), buf, 128) == 0


def test_no_device_is_an_error_not_a_fallback():
    try:
        be = qmm.Backend(0)
    except qmm.QmmError:
        return                      # no device: the product refuses instead of falling back
    be.close()
    pytest.skip("a device is present")
