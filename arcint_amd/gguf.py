"""GGUF reader: the header, metadata and tensor table of a (possibly split) GGUF file, tensor
bytes read through a memory map, and a loader that streams a tensor into a libqmm buffer.

The GGUF container (version 2 and 3, little-endian), as llama.cpp's gguf writer lays it out:

    "GGUF" | u32 version | u64 tensor count | u64 metadata count
    metadata:     string key | u32 value type | value
    tensor infos: string name | u32 n_dims | u64 ne[n_dims] (ne0 first) | u32 ggml type |
                  u64 offset into the data section
    data section: starts at the first multiple of general.alignment (default 32) past the
                  tensor infos; every tensor offset is a multiple of it

A string is a u64 byte count and UTF-8 bytes; an array value is a u32 element type, a u64
count and the elements.  The reference reads the same container (tools/mtp_fit.py:270-335).
A model split by llama.cpp's gguf-split is named <prefix>-00001-of-0000N.gguf ... -0000N-of-
0000N.gguf; every shard holds its own header and tensors and carries split.count and split.no.

The whole file is mapped, never read: the header is decoded from the map at a moving offset,
and a tensor's bytes are copied out of the map only for the range asked for.  The loader hands
GGUF block bytes to qmm_tensor_set in chunks of whole blocks (the library repacks them into its
device image).
"""
from __future__ import annotations

import os
from dataclasses import dataclass, field

import numpy as np

GGUF_MAGIC = b"GGUF"
# metadata value type -> numpy dtype (little-endian); 8 is a string, 9 an array
_VALUE_DTYPES = {0: "<u1", 1: "<i1", 2: "<u2", 3: "<i2", 4: "<u4", 5: "<i4", 6: "<f4", 7: "?",
                 10: "<u8", 11: "<i8", 12: "<f8"}
VT_STRING, VT_ARRAY = 8, 9

# ggml types: (elements per block, bytes per block) for the types a GGUF file of this path holds
GGML_TYPES = {
    0: (1, 4),          # F32
    1: (1, 2),          # F16
    2: (32, 18),        # Q4_0
    8: (32, 34),        # Q8_0
    12: (256, 144),     # Q4_K
    13: (256, 176),     # Q5_K
    14: (256, 210),     # Q6_K
    20: (32, 18),       # IQ4_NL
    23: (256, 136),     # IQ4_XS
    24: (1, 1),         # I8
    25: (1, 2),         # I16
    26: (1, 4),         # I32
    30: (1, 2),         # BF16
}


class GGUFError(ValueError):
    pass


@dataclass
class GGUFTensor:
    name: str
    ne: tuple            # ne0 first, as ggml
    type: int
    offset: int          # absolute byte offset in its file
    nbytes: int          # -1 for a ggml type this reader does not size
    path: str


@dataclass
class GGUF:
    path: str
    version: int
    kv: dict = field(default_factory=dict)
    tensors: dict = field(default_factory=dict)     # name -> GGUFTensor (all shards)
    alignment: int = 32

    def tensor(self, name: str) -> GGUFTensor:
        if name not in self.tensors:
            raise KeyError(f"no tensor {name!r} in {self.path}")
        return self.tensors[name]

    def read(self, name: str, start: int = 0, size: int | None = None) -> np.ndarray:
        """bytes [start, start + size) of a tensor's data, as uint8 (a copy of that range only)"""
        t = self.tensor(name)
        size = t.nbytes - start if size is None else size
        if start < 0 or size < 0 or start + size > t.nbytes:
            raise GGUFError(f"{name}: range [{start}, {start + size}) outside its {t.nbytes} bytes")
        if size == 0:
            return np.zeros(0, np.uint8)
        view = np.memmap(t.path, dtype=np.uint8, mode="r", offset=t.offset + start, shape=(size,))
        try:
            return np.array(view)
        finally:
            del view


def tensor_nbytes(ggml_type: int, ne) -> int:
    if ggml_type not in GGML_TYPES:
        raise GGUFError(f"ggml type {ggml_type} is not one this reader sizes")
    blck, bb = GGML_TYPES[ggml_type]
    if ne[0] % blck:
        raise GGUFError(f"ne0 = {ne[0]} is not a whole number of {blck}-element blocks")
    return int(np.prod(ne, dtype=np.int64)) // blck * bb


class _Cursor:
    """Little-endian GGUF fields decoded from a mapped file at a moving byte offset."""

    def __init__(self, buf: np.ndarray, path: str):
        self.buf, self.at, self.path = buf, 0, path

    def _span(self, n: int) -> int:
        at = self.at
        if n < 0 or at + n > self.buf.size:
            raise GGUFError(f"{self.path}: the header runs past the end of the file (byte {at} + {n})")
        self.at = at + n
        return at

    def items(self, dtype, count: int) -> np.ndarray:
        dt = np.dtype(dtype)
        at = self._span(dt.itemsize * count)
        return self.buf[at:at + dt.itemsize * count].view(dt).copy()

    def one(self, dtype):
        return self.items(dtype, 1)[0].item()

    def text(self) -> str:
        n = self.one("<u8")
        at = self._span(n)
        return bytes(self.buf[at:at + n]).decode("utf-8", "replace")

    def value(self, vtype: int):
        dt = _VALUE_DTYPES.get(vtype)
        if dt is not None:
            return self.one(dt)
        if vtype == VT_STRING:
            return self.text()
        if vtype == VT_ARRAY:
            etype, count = self.one("<u4"), self.one("<u8")
            edt = _VALUE_DTYPES.get(etype)
            if edt is not None:                                   # a numeric array: one slice of the map
                return self.items(edt, count)
            return [self.value(etype) for _ in range(count)]
        raise GGUFError(f"{self.path}: metadata value type {vtype} at byte {self.at - 4}")


def _parse(path: str) -> GGUF:
    """One GGUF file: metadata and the tensor table with absolute offsets."""
    size = os.path.getsize(path)
    if size < 24:
        raise GGUFError(f"{path}: {size} bytes is shorter than a GGUF header")
    buf = np.memmap(path, dtype=np.uint8, mode="r")
    try:
        if bytes(buf[:4]) != GGUF_MAGIC:
            raise GGUFError(f"{path}: not a GGUF file")
        cur = _Cursor(buf, path)
        cur.at = 4
        version = cur.one("<u4")
        if version not in (2, 3):
            raise GGUFError(f"{path}: GGUF version {version} (version 1's counts are 32-bit; not read)")
        n_tensors, n_kv = cur.one("<u8"), cur.one("<u8")
        out = GGUF(path=path, version=version)
        for _ in range(n_kv):
            key = cur.text()
            out.kv[key] = cur.value(cur.one("<u4"))
        align = int(out.kv.get("general.alignment", 32))
        if align <= 0 or align & (align - 1):
            raise GGUFError(f"{path}: general.alignment {align} is not a power of two")
        out.alignment = align
        table = []
        for _ in range(n_tensors):
            name = cur.text()
            n_dims = cur.one("<u4")
            if not 1 <= n_dims <= 4:
                raise GGUFError(f"{path}: tensor {name!r} has {n_dims} dimensions")
            ne = tuple(int(d) for d in cur.items("<u8", n_dims))
            table.append((name, ne + (1,) * (4 - n_dims), cur.one("<u4"), cur.one("<u8")))
        data_start = -(-cur.at // align) * align
    finally:
        del buf
    for name, ne, gtype, rel in table:
        if rel % align:
            raise GGUFError(f"{path}: tensor {name!r} offset {rel} is not a multiple of {align}")
        nbytes = tensor_nbytes(gtype, ne) if gtype in GGML_TYPES else -1
        if nbytes > 0 and data_start + rel + nbytes > size:
            raise GGUFError(f"{path}: tensor {name!r} runs past the end of the file")
        if name in out.tensors:
            raise GGUFError(f"{path}: tensor {name!r} appears twice")
        out.tensors[name] = GGUFTensor(name, ne, gtype, data_start + rel, nbytes, path)
    return out


def shard_paths(first: str, count: int) -> list[str]:
    """The file names gguf-split gives the `count` shards of a model whose first shard is
    `first` (<prefix>-00001-of-NNNNN.gguf)."""
    stem, dot, ext = first.rpartition(".")
    head, of, total = stem.rpartition("-of-")
    prefix, dash, index = head.rpartition("-")
    if not (dot and of and dash) or index != "00001" or not total.isdigit() or int(total) != count:
        raise GGUFError(f"{first}: split.count is {count} but the name is not <prefix>-00001-of-{count:05d}.{ext}")
    return [f"{prefix}-{i:05d}-of-{total}.{ext}" for i in range(1, count + 1)]


def read(path: str) -> GGUF:
    """Header, metadata and tensor table of a GGUF file; for the first shard of a split model
    the other shards' tensors are added (the metadata is the first shard's)."""
    g = _parse(path)
    count = int(g.kv.get("split.count", 1))
    if count <= 1:
        return g
    for no, shard in enumerate(shard_paths(path, count)[1:], start=1):
        if not os.path.exists(shard):
            raise GGUFError(f"{path}: shard {shard} is missing")
        part = _parse(shard)
        if int(part.kv.get("split.no", no)) != no:
            raise GGUFError(f"{shard}: split.no is {part.kv['split.no']}, its name says {no}")
        for name, t in part.tensors.items():
            if name in g.tensors:
                raise GGUFError(f"{shard}: tensor {name!r} is also in another shard")
            g.tensors[name] = t
    return g


def load_tensor(be, g: GGUF, name: str, chunk_bytes: int = 64 << 20):
    """A libqmm tensor of `name`'s type and shape in a new device buffer, its GGUF bytes
    written in chunks of whole blocks of about `chunk_bytes` (qmm_tensor_set repacks each
    range into the device image)."""
    t = g.tensor(name)
    if t.nbytes < 0:
        raise GGUFError(f"{name}: ggml type {t.type} has no size here")
    dst = be.new_tensor(t.type, t.ne)
    bb = GGML_TYPES[t.type][1]
    step = max(bb, chunk_bytes // bb * bb)
    for start in range(0, t.nbytes, step):
        be.set_tensor(dst, g.read(name, start, min(step, t.nbytes - start)), offset=start)
    return dst
