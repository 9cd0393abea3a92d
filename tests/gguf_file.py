"""A small GGUF v3 writer and tensor-table reader for tests.

The layout follows the reference's parser (src/gguf.rs:460-600): magic
"GGUF", version u32, tensor count u64, metadata count u64, metadata entries
(key string, value type u32, value), then per tensor its name string, the
dimension count u32, dimensions u64 (dims[0] = columns, the contiguous axis),
the ggml type u32 and the offset u64 relative to the data section.  The data
section starts at the header's end rounded up to `general.alignment` (32 when
absent); each tensor's absolute offset is that start plus its offset, and its
byte length is row_byte_len(dims[0]) times the other dimensions
(src/gguf.rs:988-1009).  Strings are a u64 length and the bytes.
"""
import struct
from dataclasses import dataclass

# (elements, bytes) per block of the ggml types the tests write
# (src/gguf.rs:319-342)
BLOCK = {0: (1, 4), 1: (1, 2), 6: (32, 22), 8: (32, 34), 12: (256, 144), 14: (256, 210), 30: (1, 2)}
_U32 = 4  # metadata value type of a u32


@dataclass
class TensorInfo:
    name: str
    dimensions: list
    kind: int
    absolute_offset: int
    byte_len: int


def _string(text: str) -> bytes:
    raw = text.encode()
    return struct.pack("<Q", len(raw)) + raw


def byte_len(kind: int, dimensions) -> int:
    elements, nbytes = BLOCK[kind]
    assert dimensions[0] % elements == 0
    total = dimensions[0] // elements * nbytes
    for d in dimensions[1:]:
        total *= d
    return total


def write(path, tensors, alignment: int = 32) -> None:
    """tensors: list of (name, dimensions, ggml type, encoded bytes)."""
    header = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), 1))
    header += _string("general.alignment") + struct.pack("<II", _U32, alignment)
    offsets, cursor = [], 0
    for _, dims, kind, data in tensors:
        assert len(data) == byte_len(kind, dims)
        offsets.append(cursor)
        cursor += -(-len(data) // alignment) * alignment
    for (name, dims, kind, _), off in zip(tensors, offsets):
        header += _string(name) + struct.pack("<I", len(dims))
        header += b"".join(struct.pack("<Q", d) for d in dims)
        header += struct.pack("<IQ", kind, off)
    start = -(-len(header) // alignment) * alignment
    blob = bytearray(start + cursor)
    blob[:len(header)] = header
    for (_, _, _, data), off in zip(tensors, offsets):
        blob[start + off:start + off + len(data)] = bytes(data)
    with open(path, "wb") as f:
        f.write(blob)


def read_tensors(blob) -> list:
    """The tensor table of a file written by `write` (u32 metadata only)."""
    blob = memoryview(blob)
    pos = 0

    def take(fmt):
        nonlocal pos
        values = struct.unpack_from(fmt, blob, pos)
        pos += struct.calcsize(fmt)
        return values

    def string():
        (n,) = take("<Q")
        nonlocal pos
        text = bytes(blob[pos:pos + n]).decode()
        pos += n
        return text

    assert bytes(blob[:4]) == b"GGUF"
    pos = 4
    version, count, metadata = take("<IQQ")
    assert version in (2, 3)
    alignment = 32
    for _ in range(metadata):
        key = string()
        (vtype,) = take("<I")
        assert vtype == _U32
        (value,) = take("<I")
        if key == "general.alignment":
            alignment = value
    raw = []
    for _ in range(count):
        name = string()
        (ndim,) = take("<I")
        dims = list(take("<" + "Q" * ndim))
        kind, off = take("<IQ")
        raw.append((name, dims, kind, off))
    start = -(-pos // alignment) * alignment
    return [TensorInfo(n, d, k, start + o, byte_len(k, d)) for n, d, k, o in raw]
