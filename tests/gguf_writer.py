"""TEST INFRASTRUCTURE: a minimal GGUF (version 3) writer for the reader's tests, written from
the format (magic, version, u64 counts, typed metadata, tensor infos, aligned data) with no
code shared with arcint_amd/gguf.py."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _v(t: int, v) -> bytes:
    if t in _FMT:
        return struct.pack(_FMT[t], v)
    if t == STRING:
        return _s(v)
    et, items = v
    return struct.pack("<IQ", et, len(items)) + b"".join(_v(et, i) for i in items)


def write(path, kv, tensors, version=3, alignment=None, magic=b"GGUF", pad_end=True):
    """kv: list of (key, type, value) (arrays: (elem type, list)); tensors: list of
    (name, ne tuple, ggml type, bytes).  Data offsets are laid out in order, aligned."""
    align = alignment or 32
    kv = list(kv)
    if alignment is not None:
        kv.append(("general.alignment", U32, alignment))
    head = magic + struct.pack("<IQQ", version, len(tensors), len(kv))
    head += b"".join(_s(k) + struct.pack("<I", t) + _v(t, v) for k, t, v in kv)
    infos, blobs, off = b"", [], 0
    for name, ne, ty, data in tensors:
        dims = list(ne)
        while len(dims) > 1 and dims[-1] == 1:
            dims.pop()
        infos += _s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        infos += struct.pack("<IQ", ty, off)
        blobs.append((off, bytes(data)))
        off = (off + len(data) + align - 1) // align * align
    body = head + infos
    start = (len(body) + align - 1) // align * align
    out = bytearray(body + b"\0" * (start - len(body)))
    for o, d in blobs:
        if len(out) < start + o:
            out += b"\0" * (start + o - len(out))
        out += d
    if pad_end:
        out += b"\0" * ((-len(out)) % align)
    with open(path, "wb") as f:
        f.write(out)
    return start


def random_block_bytes(ggml_type, ne, seed):
    blck, bb = {2: (32, 18), 8: (32, 34), 12: (256, 144), 14: (256, 210), 23: (256, 136), 0: (1, 4)}[ggml_type]
    n = ne[0] // blck * int(np.prod(ne[1:]))
    return np.random.default_rng(seed).integers(0, 256, n * bb, dtype=np.uint8)
