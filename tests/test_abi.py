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


def test_supports_op_views_of_quantized_weights():
    """a quantized view is taken where the base image holds its rows as whole matrices or whole
    64-row tiles (the reference's whole-slice rule, 0116-opencl-q3_K.patch:76-85, widened to
    tiles); anything else is refused with the reason"""
    L = qmm.load()
    fake = qmm.Buffer(ptr=0x1000, size=1 << 40)
    buf = C.create_string_buffer(160)
    K = 512
    _, bb = qmm.type_block(qmm.Q4_K)
    row = K // 256 * bb

    def ok(w, n=3):
        x, y = qmm.Tensor(fake, qmm.F32, (K, n, w.ne[2])), qmm.Tensor(fake, qmm.F32, (w.ne[1], n, w.ne[2]))
        return L.qmm_supports_op(None, qmm.OP_MUL_MAT, C.byref(w.c), C.byref(x.c), None, C.byref(y.c), buf, 160) == 1

    a = qmm.Tensor(fake, qmm.Q4_K, (K, 64, 3))
    assert ok(a)
    assert ok(a.view((K, 64), offset=2 * a.nb[2]))                 # slice 2
    assert ok(a.view((K, 64, 2), offset=1 * a.nb[2]))              # slices 1..2
    assert ok(a.view((K, 192)))                                    # reshape: whole tiles
    assert not ok(a.view((K, 64), offset=5 * row)) and b"whole matrices" in buf.value   # rows 5..68
    assert not ok(a.view((K, 32)))                                 # half a slice
    assert not ok(a.view((K, 64), offset=row + 7)) and b"start on a row" in buf.value
    assert not ok(a.view((K, 64, 2), offset=2 * a.nb[2])) and b"past its base" in buf.value
    b = qmm.Tensor(fake, qmm.Q4_K, (K, 100, 3))
    assert ok(b.view((K, 100), offset=b.nb[2]))
    assert not ok(b.view((K, 300)))                                # 100-row matrices are not whole tiles
    c = qmm.Tensor(fake, qmm.Q4_K, (K, 256))
    assert ok(c.view((K, 128), offset=64 * row))                   # rows 64..191: whole tiles
    assert not ok(c.view((K, 100), offset=64 * row))
    # test-backend-ops' permuted weight: [K, 1, M] seen as [K, M]
    p = qmm.Tensor(fake, qmm.Q4_K, (K, 1, 64))
    assert not ok(p.view((K, 64), nb=(bb, p.nb[2], p.nb[2], 64 * p.nb[2])))
    # MUL_MAT_ID on a run of experts of a stack
    e = qmm.Tensor(fake, qmm.Q4_K, (K, 64, 8))
    ev = e.view((K, 64, 4), offset=2 * e.nb[2])
    xe, ids, ye = (qmm.Tensor(fake, qmm.F32, (K, 1, 5)), qmm.Tensor(fake, qmm.I32, (2, 5)),
                   qmm.Tensor(fake, qmm.F32, (64, 2, 5)))
    assert L.qmm_supports_op(None, qmm.OP_MUL_MAT_ID, C.byref(ev.c), C.byref(xe.c), C.byref(ids.c), C.byref(ye.c),
                             buf, 160) == 1


def test_view_nbytes_is_ggml_nbytes():
    fake = qmm.Buffer(ptr=0x1000, size=1 << 40)
    a = qmm.Tensor(fake, qmm.Q4_K, (512, 1, 64))
    pv = a.view((512, 64), nb=(144, a.nb[2], a.nb[2], 64 * a.nb[2]))
    assert pv.nbytes == a.nbytes == 64 * 288
    assert a.view((512, 5), offset=70 * 288).nbytes == 5 * 288


def test_no_device_is_an_error_not_a_fallback():
    try:
        be = qmm.Backend(0)
    except qmm.QmmError:
        return                      # no device: the product refuses instead of falling back
    be.close()
    pytest.skip("a device is present")


def test_moe_ffn_args_layout():
    """qmm_moe_ffn_args as the C compiler lays it out (gcc on the header) equals the binding's
    ctypes structure, field by field"""
    import shutil
    import subprocess
    import tempfile
    if not shutil.which("gcc"):
        pytest.skip("no gcc")
    fields = [f for f, _ in qmm.CMoeFfn._fields_]
    body = "".join(f'printf("%zu\\n", offsetof(qmm_moe_ffn_args, {f}));' for f in fields)
    src = ('#include "qmm.h"\n#include <stddef.h>\n#include <stdio.h>\n'
           f'int main(void) {{ printf("%zu\\n", sizeof(qmm_moe_ffn_args)); {body} return 0; }}\n')
    with tempfile.TemporaryDirectory() as d:
        c, exe = os.path.join(d, "l.c"), os.path.join(d, "l")
        open(c, "w").write(src)
        subprocess.run(["gcc", "-I" + os.path.join(ROOT, "include"), c, "-o", exe], check=True)
        got = [int(v) for v in subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split()]
    assert got == [C.sizeof(qmm.CMoeFfn)] + [getattr(qmm.CMoeFfn, f).offset for f in fields]
