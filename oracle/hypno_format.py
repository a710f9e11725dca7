"""CPU restatement of hypno's `.hypno` file format (crates/hypno/src/format.rs,
loader.rs, sft_convert.rs).

TEST INFRASTRUCTURE ONLY: the checker for the library's model reader
(hypno_hip_model_*).  Only tests/ and bench.py's fixture writer use it; the
product package ``hypno_amd`` never does.

read(buf)   restates HypnoModel::open after the mapping (loader.rs:44-134):
            the same fields, checks and check order, raising FormatErr with
            the FormatError variant (format.rs:109-131) and its fields.  One
            deliberate difference: a tensor name whose bytes run past the end
            of the buffer is BufferTooShort here (the reference slices it
            without a bounds check, loader.rs:96-97).
write(...)  restates the converter's layout (sft_convert.rs:121-289): header,
            metadata pairs, tensor table, zero padding to the 64-byte data
            start, then each payload at a 64-byte-aligned offset, zero-padded
            to the next 64-byte boundary.

Pinned by: the reference's own loader test (loader.rs:224-319, rebuilt byte
for byte as tests/golden/loader_test.hypno by tests/golden/make_hypno_fixture.py
and checked against that test's assertions), the converter test's size rule
(sft_convert.rs:430-457: 8192 Q4_0 elements -> 4608 bytes) and layout
invariants (every payload offset a multiple of 64; data start = the table end
rounded up to 64).
"""
from __future__ import annotations

import dataclasses
import struct
from typing import List, Sequence, Tuple

MAGIC = b"HYPN"        # format.rs:4
FORMAT_VERSION = 1     # format.rs:7
ALIGNMENT = 64         # format.rs:10
DTYPES = (0, 1, 2, 3)  # FP32, FP16, Q8_0, Q4_0 (dtype.rs:4-15)


class FormatErr(Exception):
    """FormatError variant name plus its fields, e.g. ("BufferTooShort", 40, 33)."""

    def __init__(self, kind: str, *fields):
        super().__init__(kind, *fields)
        self.kind = kind
        self.fields = fields


@dataclasses.dataclass(frozen=True)
class Tensor:
    name: str
    shape: Tuple[int, ...]
    dtype: int
    offset: int
    data_len: int

    @property
    def ndim(self) -> int:
        return len(self.shape)


@dataclasses.dataclass(frozen=True)
class Manifest:
    version: int
    metadata_kv_count: int
    tensor_count: int
    metadata: List[Tuple[str, str]]
    tensors: List[Tensor]


def data_bytes(dtype: int, n_elems: int) -> int:
    """DType::data_bytes (dtype.rs:58-70)."""
    if dtype == 0:
        return 4 * n_elems
    if dtype == 1:
        return 2 * n_elems
    return -(-n_elems // 32) * (34 if dtype == 2 else 18)


def effective_dtype(target: int, n_elems: int) -> int:
    """sft_convert.rs:11-17: tensors of <= 4096 elements stay FP32 when quantizing."""
    return 0 if n_elems <= 4096 and target not in (0, 1) else target


def _utf8(b: bytes) -> str:
    try:
        return b.decode("utf-8", errors="strict")
    except UnicodeDecodeError as e:
        raise FormatErr("Utf8", e.start) from None


def read(buf: bytes) -> Manifest:
    size = len(buf)
    if size < 16:
        raise FormatErr("BufferTooShort", 16, size)
    magic = bytes(buf[0:4])
    version, kv_count, tensor_count = struct.unpack_from("<III", buf, 4)
    if magic != MAGIC:
        raise FormatErr("InvalidMagic", magic)
    if version != FORMAT_VERSION:
        raise FormatErr("UnsupportedVersion", version)
    cur = 16

    def u32():
        nonlocal cur
        if cur + 4 > size:
            raise FormatErr("BufferTooShort", cur + 4, size)
        v = struct.unpack_from("<I", buf, cur)[0]
        cur += 4
        return v

    def u64():
        nonlocal cur
        if cur + 8 > size:
            raise FormatErr("BufferTooShort", cur + 8, size)
        v = struct.unpack_from("<Q", buf, cur)[0]
        cur += 8
        return v

    def string(n):
        nonlocal cur
        if cur + n > size:
            raise FormatErr("BufferTooShort", cur + n, size)
        s = _utf8(bytes(buf[cur:cur + n]))
        cur += n
        return s

    metadata = []
    for _ in range(kv_count):
        k = string(u32())
        v = string(u32())
        metadata.append((k, v))
    tensors = []
    for _ in range(tensor_count):
        name = string(u32())
        ndim = u32()
        shape = tuple(u64() for _ in range(ndim))
        dtype = u32()
        if dtype not in DTYPES:
            raise FormatErr("UnknownDType", dtype)
        offset = u64()
        data_len = u64()
        if offset > size or offset + data_len > size:
            raise FormatErr("InvalidOffset", offset, size)
        tensors.append(Tensor(name, shape, dtype, offset, data_len))
    return Manifest(version, kv_count, tensor_count, metadata, tensors)


def _align(x: int) -> int:
    return (x + ALIGNMENT - 1) // ALIGNMENT * ALIGNMENT


def write(metadata: Sequence[Tuple[str, str]],
          tensors: Sequence[Tuple[str, Sequence[int], int, bytes]]) -> bytes:
    """Serialise (name, shape, dtype, payload) tensors in the given order."""
    head = bytearray(struct.pack("<4sIII", MAGIC, FORMAT_VERSION, len(metadata), len(tensors)))
    for k, v in metadata:
        kb, vb = k.encode(), v.encode()
        head += struct.pack("<I", len(kb)) + kb + struct.pack("<I", len(vb)) + vb
    table_size = sum(4 + len(n.encode()) + 4 + 8 * len(s) + 4 + 8 + 8 for n, s, _, _ in tensors)
    data_start = _align(len(head) + table_size)
    offsets, cur = [], data_start
    for _, _, _, payload in tensors:
        offsets.append(cur)
        cur = _align(cur + len(payload))
    for (name, shape, dtype, payload), off in zip(tensors, offsets):
        nb = name.encode()
        head += struct.pack("<I", len(nb)) + nb + struct.pack("<I", len(shape))
        head += b"".join(struct.pack("<Q", d) for d in shape)
        head += struct.pack("<IQQ", dtype, off, len(payload))
    out = head + bytes(data_start - len(head))
    for (_, _, _, payload), off in zip(tensors, offsets):
        out += bytes(off - len(out)) + payload
        out += bytes(_align(len(out)) - len(out))
    return bytes(out)
