"""Writers of small GGUF files and llamafile (ZIP) wrappers for the tests.

The layouts follow the reference's test builders: buildMinimalGguf and
buildLlamafile (GgufReaderTest.java:441-574) and the large-stub llamafile of
GgufReaderTest.java:706-794; ``gguf_bytes`` generalises the first to metadata
of every value type and several tensors, ``zip64_llamafile`` adds the ZIP64
records that findGgufOffsetInZip resolves (GgufReader.java:850-880,
1136-1154).
"""
from __future__ import annotations

import struct

import numpy as np

MAGIC = 0x46554747
ALIGN = 32

UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_FMT = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
        UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}


def _str(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == STRING:
        return _str(v)
    if vtype == BOOL:
        return struct.pack("<B", 1 if v else 0)
    if vtype == ARRAY:
        et, items = v
        return struct.pack("<iQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    return struct.pack(_FMT[vtype], v)


def gguf_bytes(metadata=(), tensors=(), version: int = 3) -> bytes:
    """metadata: (key, vtype, value) triples (ARRAY value = (elem_type, items));
    tensors: (name, dims, ggml_type, data bytes) with dims in GGUF order
    (dims[0] = the row length).  Tensor data is laid out in order, each at a
    32-byte aligned offset of the data section."""
    out = bytearray(struct.pack("<IiQQ", MAGIC, version, len(tensors), len(metadata)))
    for key, vt, v in metadata:
        out += _str(key) + struct.pack("<i", vt) + _value(vt, v)
    offs, at = [], 0
    for _, _, _, data in tensors:
        offs.append(at)
        at = (at + len(data) + ALIGN - 1) // ALIGN * ALIGN
    for (name, dims, t, _), off in zip(tensors, offs):
        out += _str(name) + struct.pack("<i", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<iQ", t, off)
    out += bytes((-len(out)) % ALIGN)
    base = len(out)
    for (_, _, _, data), off in zip(tensors, offs):
        out += bytes(base + off - len(out)) + bytes(data)
    return bytes(out)


def minimal_gguf(name: str, ggml_type: int, nelems: int, data: bytes) -> bytes:
    """buildMinimalGguf (GgufReaderTest.java:441-491): version 3, no metadata,
    one 1-D tensor at offset 0."""
    return gguf_bytes((), [(name, [nelems], ggml_type, data)])


def f32_bytes(values) -> bytes:
    return np.asarray(values, dtype="<f4").tobytes()


STUB = b"MZqFpD" + bytes(26)


def _local_header(fn: bytes, size: int, extra: bytes = b"", size32=None) -> bytes:
    s = size if size32 is None else size32
    return struct.pack("<IHHHHHIIIHH", 0x04034B50, 20, 0, 0, 0, 0, 0, s, s, len(fn), len(extra)) + fn + extra


def _cd_entry(fn: bytes, size: int, lho: int, extra: bytes = b"", size32=None) -> bytes:
    s = size if size32 is None else size32
    return struct.pack("<IHHHHHHIIIHHHHHII", 0x02014B50, 20, 20, 0, 0, 0, 0, 0, s, s, len(fn), len(extra), 0, 0, 0,
                       0, lho) + fn + extra


def _eocd(cd_size: int, cd_off: int, entries: int = 1) -> bytes:
    return struct.pack("<IHHHHIIH", 0x06054B50, 0, 0, entries, entries, cd_size, cd_off, 0)


def llamafile(entry: str, gguf: bytes, stub: bytes = STUB, overlay: bytes = b"", others=()) -> bytes:
    """buildLlamafile (GgufReaderTest.java:502-574): [stub][local header + GGUF]
    [central directory][EOCD], optionally preceded by other stored entries and
    followed by an overlay (GgufReaderTest.java:666-700)."""
    body, cd = bytearray(stub), bytearray()
    for name, data in list(others) + [(entry, gguf)]:
        fn = name.encode()
        lho = len(body)
        body += _local_header(fn, len(data)) + data
        cd += _cd_entry(fn, len(data), lho)
    n = len(others) + 1
    return bytes(body + cd + _eocd(len(cd), len(body), n) + overlay)


def zip64_llamafile(entry: str, gguf: bytes, stub: bytes = STUB) -> bytes:
    """A ZIP64 llamafile: the EOCD holds 0xFFFFFFFF for the directory size and
    offset, resolved through the ZIP64 locator and record, and the directory
    entry's local-header offset is 0xFFFFFFFF with the real one in its ZIP64
    extra field (id 1: uncompressed size, compressed size, offset)."""
    fn = entry.encode()
    lho = len(stub)
    body = bytearray(stub) + _local_header(fn, len(gguf)) + gguf
    extra = struct.pack("<HHQQQ", 0x0001, 24, len(gguf), len(gguf), lho)
    cd = _cd_entry(fn, len(gguf), 0xFFFFFFFF, extra, size32=0xFFFFFFFF)
    cd_off = len(body)
    z64_pos = cd_off + len(cd)
    z64 = struct.pack("<IQHHIIQQQQ", 0x06064B50, 44, 45, 45, 0, 0, 1, 1, len(cd), cd_off)
    loc = struct.pack("<IIQI", 0x07064B50, 0, z64_pos, 1)
    eocd = struct.pack("<IHHHHIIH", 0x06054B50, 0, 0, 0xFFFF, 0xFFFF, 0xFFFFFFFF, 0xFFFFFFFF, 0)
    return bytes(body + cd + z64 + loc + eocd)


def big_stub_llamafile(entry: str, gguf: bytes, stub_len: int = 1_200_000, overlay_len: int = 70_000) -> bytes:
    """GgufReaderTest.java:706-794: a 1.2 MB zero stub (beyond one 1 MiB scan
    window) and a 70 000-byte overlay after the EOCD, so that only the forward
    scan finds the entry."""
    stub = bytearray(stub_len)
    stub[:4] = b"MZqF"
    return llamafile(entry, gguf, stub=bytes(stub), overlay=bytes(overlay_len))
