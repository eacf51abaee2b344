"""GGUF container: the on-disk format that feeds the quantized matvecs.

Mirrors the reference's parser, crates/modgrad-device/src/kfd/gguf.rs:9-244
and :665-694 -- `GgmlType` with its block sizes, `TensorInfo`, `MetaValue`
accessors, `GgufFile.parse` and its error messages -- over a seekable binary
stream. Tensor data is not read at parse time; `GgufFile.open` memory-maps
the file and `tensor_bytes` returns a zero-copy view of one tensor.

Conventions (as the reference uses them, rocm_gemma.rs:174-178): a weight's
dims[0] is its input width K and dims[1] its output count N, so a row-aligned
Q4_K matrix is N rows of K/256 blocks.

One deliberate difference: the data section starts at the header end rounded
up to `general.alignment` when the file sets it (the GGUF specification), and
to 32 bytes otherwise. The reference always uses 32 (gguf.rs:207-209); the
two agree on every file that leaves the key unset or sets it to 32.

`write_gguf` is an addition (the reference only reads GGUF): it writes GGUF
v3 with tensor data aligned like llama.cpp's writer, for fixtures and export.
"""
from __future__ import annotations

import mmap
import os
import struct
from dataclasses import dataclass, field
from enum import IntEnum

import numpy as np


class GgufError(ValueError):
    """A malformed or unsupported file (the reference's Err(String))."""


class GgmlType(IntEnum):
    """Tensor element types (gguf.rs:9-43); other ids parse as UNKNOWN."""
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q8_1 = 9
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    Q8_K = 15
    IQ2_XXS = 16
    BF16 = 30
    UNKNOWN = -1


# (block bytes, block elements), gguf.rs:48-67; unknown types are (0, 1)
_BLOCK = {
    GgmlType.F32: (4, 1), GgmlType.F16: (2, 1), GgmlType.BF16: (2, 1),
    GgmlType.Q4_0: (18, 32), GgmlType.Q4_1: (20, 32), GgmlType.Q5_0: (22, 32),
    GgmlType.Q5_1: (24, 32), GgmlType.Q8_0: (34, 32), GgmlType.Q8_1: (36, 32),
    GgmlType.Q2_K: (84, 256), GgmlType.Q3_K: (110, 256), GgmlType.Q4_K: (144, 256),
    GgmlType.Q5_K: (176, 256), GgmlType.Q6_K: (210, 256), GgmlType.Q8_K: (292, 256),
}


def ggml_type(v: int) -> GgmlType:
    try:
        return GgmlType(v)
    except ValueError:
        return GgmlType.UNKNOWN


def block_size(t: GgmlType) -> tuple[int, int]:
    return _BLOCK.get(t, (0, 1))


def data_size(t: GgmlType, n_elements: int) -> int:
    """Bytes of n_elements of type t, whole blocks (gguf.rs:71-75)."""
    bb, be = block_size(t)
    return (n_elements + be - 1) // be * bb


@dataclass
class TensorInfo:
    name: str
    dims: list[int]
    dtype: GgmlType
    offset: int          # from the data section start
    dtype_id: int = -1   # the raw type id (kept for UNKNOWN types)

    def n_elements(self) -> int:
        n = 1
        for d in self.dims:
            n *= d
        return max(n, 1)

    def data_bytes(self) -> int:
        return data_size(self.dtype, self.n_elements())


# value types (gguf.rs:665-694)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
           BOOL: "<B", U64: "<Q", I64: "<q", F64: "<d"}


@dataclass
class MetaValue:
    """A typed metadata value; `value` is a Python scalar, str or list of
    MetaValue (arrays)."""
    vtype: int
    value: object

    def as_u32(self):
        """U32, or I32 / U64 cast to u32 (gguf.rs:117-124)."""
        if self.vtype == U32:
            return self.value
        if self.vtype in (I32, U64):
            return int(self.value) & 0xFFFFFFFF
        return None

    def as_f32(self):
        if self.vtype == F32:
            return self.value
        if self.vtype == F64:
            return float(np.float32(self.value))
        return None

    def as_str(self):
        return self.value if self.vtype == STRING else None

    def as_bool_array(self):
        if self.vtype != ARRAY:
            return None
        out = []
        for v in self.value:
            if v.vtype != BOOL:
                return None
            out.append(v.value)
        return out

    def as_list(self):
        """Array elements as plain Python values (None if not an array)."""
        if self.vtype != ARRAY:
            return None
        return [v.value for v in self.value]


MAX_STRING = 1_000_000  # gguf.rs:240


class _Reader:
    def __init__(self, f):
        self.f = f

    def exact(self, n: int) -> bytes:
        b = self.f.read(n)
        if len(b) != n:
            raise GgufError("failed to fill whole buffer")
        return b

    def u32(self) -> int:
        return struct.unpack("<I", self.exact(4))[0]

    def u64(self) -> int:
        return struct.unpack("<Q", self.exact(8))[0]

    def string(self) -> str:
        n = self.u64()
        if n > MAX_STRING:
            raise GgufError("string too long")
        try:
            return self.exact(n).decode("utf-8")
        except UnicodeDecodeError as e:
            raise GgufError(str(e)) from None

    def value(self, vtype: int) -> MetaValue:
        if vtype in _SCALAR:
            fmt = _SCALAR[vtype]
            v = struct.unpack(fmt, self.exact(struct.calcsize(fmt)))[0]
            if vtype == BOOL:
                v = v != 0
            return MetaValue(vtype, v)
        if vtype == STRING:
            return MetaValue(STRING, self.string())
        if vtype == ARRAY:
            atype = self.u32()
            n = self.u64()
            return MetaValue(ARRAY, [self.value(atype) for _ in range(n)])
        raise GgufError(f"unknown GGUF value type {vtype}")


@dataclass
class GgufFile:
    metadata: dict[str, MetaValue] = field(default_factory=dict)
    tensors: dict[str, TensorInfo] = field(default_factory=dict)
    tensor_list: list[str] = field(default_factory=list)
    data_offset: int = 0
    version: int = 3
    _map: object = None  # the memory map of an opened file

    @classmethod
    def parse(cls, f) -> "GgufFile":
        """Metadata and tensor infos from a binary stream positioned at the
        file start (gguf.rs:153-211). Tensor data is not read."""
        r = _Reader(f)
        if r.exact(4) != b"GGUF":
            raise GgufError("not a GGUF file")
        version = r.u32()
        if version < 2 or version > 3:
            raise GgufError(f"unsupported GGUF version {version}")
        n_tensors = r.u64()
        n_kv = r.u64()
        g = cls(version=version)
        for _ in range(n_kv):
            key = r.string()
            g.metadata[key] = r.value(r.u32())
        for _ in range(n_tensors):
            name = r.string()
            n_dims = r.u32()
            dims = [r.u64() for _ in range(n_dims)]
            tid = r.u32()
            offset = r.u64()
            g.tensor_list.append(name)
            g.tensors[name] = TensorInfo(name, dims, ggml_type(tid), offset, tid)
        align = 32
        a = g.metadata.get("general.alignment")
        if a is not None and a.as_u32():
            align = a.as_u32()
        pos = f.tell()
        g.data_offset = (pos + align - 1) // align * align
        return g

    @classmethod
    def open(cls, path: str) -> "GgufFile":
        """Parse `path` and keep a read-only memory map of it for
        `tensor_bytes` (5 GB of weights cost no memory until touched)."""
        with open(path, "rb") as fh:
            g = cls.parse(fh)
            g._map = mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ) if os.path.getsize(path) else b""
        return g

    def meta(self, key: str):
        return self.metadata.get(key)

    def architecture(self):
        v = self.meta("general.architecture")
        return v.as_str() if v else None

    def meta_u32(self, key: str):
        v = self.meta(key)
        return v.as_u32() if v else None

    def meta_f32(self, key: str):
        v = self.meta(key)
        return v.as_f32() if v else None

    def tensor_file_offset(self, name: str):
        """Absolute byte position of a tensor's data (gguf.rs:233-235)."""
        t = self.tensors.get(name)
        return None if t is None else self.data_offset + t.offset

    def tensor_bytes(self, name: str) -> memoryview:
        """Zero-copy view of a tensor's bytes in the memory-mapped file."""
        if self._map is None:
            raise GgufError("tensor_bytes needs a file opened with GgufFile.open")
        t = self.tensors[name]
        start = self.data_offset + t.offset
        end = start + t.data_bytes()
        if end > len(self._map):
            raise GgufError(f"tensor {name} runs past the end of the file")
        return memoryview(self._map)[start:end]

    def close(self) -> None:
        if isinstance(self._map, mmap.mmap):
            self._map.close()
        self._map = None


# ------------------------------------------------------------------ writer --

def _pack_string(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _pack_value(vtype: int, value) -> bytes:
    if vtype in _SCALAR:
        return struct.pack(_SCALAR[vtype], int(bool(value)) if vtype == BOOL else value)
    if vtype == STRING:
        return _pack_string(value)
    if vtype == ARRAY:
        atype, items = value
        return struct.pack("<IQ", atype, len(items)) + b"".join(_pack_value(atype, v) for v in items)
    raise GgufError(f"unknown GGUF value type {vtype}")


def write_gguf(path: str, metadata: list[tuple[str, int, object]],
               tensors: list[tuple[str, list[int], int, bytes]], alignment: int = 32) -> None:
    """Write GGUF v3. metadata: (key, vtype, value), arrays as
    (key, ARRAY, (elem_type, [values])); tensors: (name, dims, ggml type id,
    bytes). Each tensor's data starts at a multiple of `alignment` from the
    data section (also recorded as general.alignment when it is not 32)."""
    kv = list(metadata)
    if alignment != 32 and not any(k == "general.alignment" for k, _, _ in kv):
        kv.append(("general.alignment", U32, alignment))
    head = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kv)))
    for key, vtype, value in kv:
        head += _pack_string(key) + struct.pack("<I", vtype) + _pack_value(vtype, value)
    offsets, off = [], 0
    for name, dims, tid, data in tensors:
        off = (off + alignment - 1) // alignment * alignment
        offsets.append(off)
        off += len(data)
    for (name, dims, tid, data), o in zip(tensors, offsets):
        head += _pack_string(name) + struct.pack("<I", len(dims))
        head += b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", tid, o)
    data_start = (len(head) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * (data_start - len(head)))
        pos = 0
        for (name, dims, tid, data), o in zip(tensors, offsets):
            f.write(b"\0" * (o - pos))
            f.write(data)
            pos = o + len(data)
