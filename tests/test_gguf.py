"""GGUF reader (arcint_amd/gguf.py) against files written from the format by tests/gguf_writer.py,
without a device."""
import os
import struct

import numpy as np
import pytest

from arcint_amd import gguf
import gguf_writer as W

TYPES = [(2, (64, 3)), (8, (96, 2)), (12, (512, 3, 2)), (14, (256, 5)), (23, (256, 1, 3)), (0, (7, 5))]


def test_metadata_of_every_value_type(tmp_path):
    kv = [("a.u8", W.U8, 200), ("a.i8", W.I8, -5), ("a.u16", W.U16, 60000), ("a.i16", W.I16, -30000),
          ("a.u32", W.U32, 4000000000), ("a.i32", W.I32, -2000000000), ("a.f32", W.F32, 1.5),
          ("a.bool", W.BOOL, True), ("a.str", W.STRING, "héllo"), ("a.u64", W.U64, 2 ** 63 + 5),
          ("a.i64", W.I64, -(2 ** 62)), ("a.f64", W.F64, 2.0 ** -40),
          ("a.ints", W.ARRAY, (W.I32, [3, -1, 7])), ("a.strs", W.ARRAY, (W.STRING, ["x", "", "yz"])),
          ("a.nest", W.ARRAY, (W.ARRAY, [(W.U8, [1, 2]), (W.U8, [])]))]
    p = tmp_path / "m.gguf"
    W.write(p, kv, [])
    g = gguf.read(str(p))
    assert g.version == 3 and g.tensors == {}
    for k, t, v in kv:
        got = g.kv[k]
        if t == W.ARRAY and v[0] == W.ARRAY:
            assert [list(x) for x in got] == [[1, 2], []]
        elif t == W.ARRAY:
            assert list(got) == v[1]
        elif t == W.F32:
            assert got == np.float32(v)
        else:
            assert got == v


@pytest.mark.parametrize("alignment", [None, 64, 4096])
def test_tensor_table_offsets_and_bytes(tmp_path, alignment):
    tensors = [(f"t{i}", ne, ty, W.random_block_bytes(ty, ne, seed=i)) for i, (ty, ne) in enumerate(TYPES)]
    p = tmp_path / "t.gguf"
    start = W.write(p, [("general.name", W.STRING, "x")], tensors, alignment=alignment)
    g = gguf.read(str(p))
    assert g.alignment == (alignment or 32)
    raw = p.read_bytes()
    for name, ne, ty, data in tensors:
        t = g.tensor(name)
        assert t.type == ty and t.ne == tuple(ne) + (1,) * (4 - len(ne)) and t.nbytes == len(data)
        assert t.offset >= start and t.offset % g.alignment == 0
        assert np.array_equal(g.read(name), data)
        assert bytes(raw[t.offset:t.offset + t.nbytes]) == bytes(data)
        # partial ranges
        assert np.array_equal(g.read(name, 5, 17), data[5:22])
        assert np.array_equal(g.read(name, len(data) - 3), data[-3:])
        with pytest.raises(gguf.GGUFError):
            g.read(name, len(data) - 3, 4)


def test_split_model(tmp_path):
    t = [(f"w{i}", (256, 2), 12, W.random_block_bytes(12, (256, 2), seed=40 + i)) for i in range(5)]
    base = str(tmp_path / "model")
    W.write(base + "-00001-of-00003.gguf", [("split.count", W.U16, 3), ("general.arch", W.STRING, "q")], t[:2])
    W.write(base + "-00002-of-00003.gguf", [("split.count", W.U16, 3)], t[2:4])
    W.write(base + "-00003-of-00003.gguf", [("split.count", W.U16, 3)], t[4:])
    g = gguf.read(base + "-00001-of-00003.gguf")
    assert sorted(g.tensors) == [f"w{i}" for i in range(5)] and g.kv["general.arch"] == "q"
    for name, ne, ty, data in t:
        assert np.array_equal(g.read(name), data)
    assert g.tensor("w3").path.endswith("-00002-of-00003.gguf")
    os.remove(base + "-00003-of-00003.gguf")
    with pytest.raises(gguf.GGUFError):
        gguf.read(base + "-00001-of-00003.gguf")


def test_rejects_malformed_files(tmp_path):
    p = tmp_path / "bad.gguf"
    W.write(p, [], [], magic=b"GGML")
    with pytest.raises(gguf.GGUFError):
        gguf.read(str(p))
    W.write(p, [], [], version=1)
    with pytest.raises(gguf.GGUFError):
        gguf.read(str(p))
    d = W.random_block_bytes(2, (64, 4), seed=1)
    W.write(p, [], [("w", (64, 4), 2, d)], pad_end=False)
    p.write_bytes(p.read_bytes()[:-1])                         # the last tensor cut short
    with pytest.raises(gguf.GGUFError):
        gguf.read(str(p))
    W.write(p, [], [("w", (60, 4), 2, d[:18 * 4])])             # ne0 not whole Q4_0 blocks
    with pytest.raises(gguf.GGUFError):
        gguf.read(str(p))
    W.write(p, [("x", W.STRING, "abc")], [])
    b = bytearray(p.read_bytes())
    struct.pack_into("<I", b, 4 + 4 + 16 + 8 + 1, 99)          # the value type of key "x"
    p.write_bytes(bytes(b))
    with pytest.raises(gguf.GGUFError):
        gguf.read(str(p))


def test_split_numbering_checked(tmp_path):
    """each shard's split.no must match its name, and a split model is opened by its first
    shard, named <prefix>-00001-of-NNNNN.gguf"""
    t = [(f"w{i}", (256, 2), 12, W.random_block_bytes(12, (256, 2), seed=60 + i)) for i in range(2)]
    base = str(tmp_path / "m")
    W.write(base + "-00001-of-00002.gguf", [("split.count", W.U16, 2), ("split.no", W.U16, 0)], t[:1])
    W.write(base + "-00002-of-00002.gguf", [("split.count", W.U16, 2), ("split.no", W.U16, 1)], t[1:])
    g = gguf.read(base + "-00001-of-00002.gguf")
    assert sorted(g.tensors) == ["w0", "w1"]
    assert gguf.shard_paths(base + "-00001-of-00002.gguf", 2)[1] == base + "-00002-of-00002.gguf"
    W.write(base + "-00002-of-00002.gguf", [("split.count", W.U16, 2), ("split.no", W.U16, 0)], t[1:])
    with pytest.raises(gguf.GGUFError):
        gguf.read(base + "-00001-of-00002.gguf")
    W.write(str(tmp_path / "solo.gguf"), [("split.count", W.U16, 2)], t[:1])
    with pytest.raises(gguf.GGUFError):
        gguf.read(str(tmp_path / "solo.gguf"))
