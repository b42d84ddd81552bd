"""GGUF reader: the header, metadata and tensor table of a (possibly split) GGUF file, tensor
bytes read through a memory map, and a loader that streams a tensor into a libqmm buffer.

Format as the reference reads it (tools/mtp_fit.py:270-335, read_gguf_header /
find_gguf_tensor): "GGUF", version (>= 2), tensor count and metadata count (u64), the
metadata as (string key, u32 type, value) with strings as u64 length + UTF-8 bytes and
arrays as (u32 element type, u64 count, elements); then per tensor its name, u32 dimension
count, u64 dims (ne0 first), u32 ggml type and u64 offset relative to the data section,
which starts at the next multiple of `general.alignment` (32 by default).  A split model
(`name-00001-of-0000N.gguf`) keeps each tensor in one of its shards.

The loader hands GGUF block bytes to qmm_tensor_set in chunks of whole blocks (the library
repacks them into its device image); bytes never pass through a whole-file copy in host
memory.
"""
from __future__ import annotations

import os
import re
import struct
from dataclasses import dataclass, field

import numpy as np

GGUF_MAGIC = b"GGUF"
# metadata value types
_FIXED = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
T_STRING, T_ARRAY = 8, 9

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
    nbytes: int
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
        mm = np.memmap(t.path, dtype=np.uint8, mode="r", offset=t.offset + start, shape=(size,)) if size else None
        out = np.array(mm, copy=True) if size else np.zeros(0, np.uint8)
        del mm
        return out


def tensor_nbytes(ggml_type: int, ne) -> int:
    if ggml_type not in GGML_TYPES:
        raise GGUFError(f"ggml type {ggml_type} is not one this reader sizes")
    blck, bb = GGML_TYPES[ggml_type]
    if ne[0] % blck:
        raise GGUFError(f"ne0 = {ne[0]} is not a whole number of {blck}-element blocks")
    n = ne[0] // blck
    for d in ne[1:]:
        n *= d
    return int(n * bb)


class _Reader:
    def __init__(self, f):
        self.f = f

    def take(self, n: int) -> bytes:
        b = self.f.read(n)
        if len(b) != n:
            raise GGUFError("truncated GGUF file")
        return b

    def u32(self) -> int:
        return struct.unpack("<I", self.take(4))[0]

    def u64(self) -> int:
        return struct.unpack("<Q", self.take(8))[0]

    def string(self) -> str:
        return self.take(self.u64()).decode("utf-8", "replace")

    def value(self, t: int):
        if t in _FIXED:
            fmt = _FIXED[t]
            return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]
        if t == T_STRING:
            return self.string()
        if t == T_ARRAY:
            et, n = self.u32(), self.u64()
            if et in _FIXED:                                      # numeric arrays in one read
                fmt = _FIXED[et]
                dt = np.dtype(fmt.replace("?", "b1"))
                return np.frombuffer(self.take(dt.itemsize * n), dtype=dt).copy()
            return [self.value(et) for _ in range(n)]
        raise GGUFError(f"GGUF metadata value type {t}")


def _read_one(path: str) -> GGUF:
    with open(path, "rb") as f:
        if f.read(4) != GGUF_MAGIC:
            raise GGUFError(f"{path}: not a GGUF file")
        r = _Reader(f)
        version = r.u32()
        if version < 2:
            raise GGUFError(f"{path}: GGUF version {version} (counts of version 1 are 32-bit; not read)")
        n_tensors, n_kv = r.u64(), r.u64()
        g = GGUF(path=path, version=version)
        for _ in range(n_kv):
            key = r.string()
            g.kv[key] = r.value(r.u32())
        g.alignment = int(g.kv.get("general.alignment", 32))
        if g.alignment <= 0 or g.alignment & (g.alignment - 1):
            raise GGUFError(f"{path}: general.alignment {g.alignment} is not a power of two")
        infos = []
        for _ in range(n_tensors):
            name = r.string()
            nd = r.u32()
            if nd > 4:
                raise GGUFError(f"{path}: tensor {name!r} has {nd} dimensions")
            dims = tuple(r.u64() for _ in range(nd))
            ty, off = r.u32(), r.u64()
            infos.append((name, dims, ty, off))
        pos = f.tell()
        data = (pos + g.alignment - 1) // g.alignment * g.alignment
        size = os.fstat(f.fileno()).st_size
    for name, dims, ty, off in infos:
        ne = tuple(dims) + (1,) * (4 - len(dims))
        nbytes = tensor_nbytes(ty, ne) if ty in GGML_TYPES else -1
        if off % g.alignment:
            raise GGUFError(f"{path}: tensor {name!r} offset {off} is not aligned to {g.alignment}")
        if nbytes >= 0 and data + off + nbytes > size:
            raise GGUFError(f"{path}: tensor {name!r} runs past the end of the file")
        if name in g.tensors:
            raise GGUFError(f"{path}: tensor {name!r} appears twice")
        g.tensors[name] = GGUFTensor(name, ne, ty, data + off, nbytes, path)
    return g


def read(path: str) -> GGUF:
    """Header, metadata and tensor table of a GGUF file; for the first shard of a split model
    (`-00001-of-0000N`) the other shards' tensors are added (metadata from the first)."""
    g = _read_one(path)
    n = int(g.kv.get("split.count", 1))
    m = re.search(r"-00001-of-(\d+)", path)
    if n > 1 and m:
        for k in range(2, n + 1):
            shard = path[:m.start()] + "-%05d-of-%s" % (k, m.group(1)) + path[m.end():]
            if not os.path.exists(shard):
                raise GGUFError(f"{path}: shard {shard} is missing")
            s = _read_one(shard)
            for name, t in s.tensors.items():
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
    blck, bb = GGML_TYPES[t.type]
    step = max(bb, chunk_bytes // bb * bb)
    for start in range(0, t.nbytes, step):
        size = min(step, t.nbytes - start)
        be.set_tensor(dst, g.read(name, start, size), offset=start)
    return dst
