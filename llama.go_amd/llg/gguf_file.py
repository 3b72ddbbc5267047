"""GGUF files: the reader of gguf/reader.go and a writer for synthetic models.

Reader (gguf.Open, reader.go:27-115): little-endian header {magic "GGUF",
version 1..3, u64 tensor count, u64 metadata count}, then the metadata pairs
(u64-length string key, u32 value type, value; arrays are u32 element type +
u64 count), then the tensor descriptors (name, u32 n_dims <= 4, u64 dims
innermost first, u32 GGML type, u64 offset relative to the data section).  The
data section starts at the next multiple of 32 bytes (reader.go:93-99: the
reference uses 32 whatever general.alignment says), and offsets are made
absolute by adding its start.  Strings above 1 << 24 bytes and arrays above
1 << 20 elements are errors, as in reader.go:279-281 and :341-343.  The
reference reads every version with u64 counts and lengths; so does this one.

Writer: the inverse, for version 3, each tensor's data at a 32-byte aligned
offset within the data section, so that the file is one the reference's
reader accepts.  Tensor data is read back with numpy memory maps, so a large
model never needs to fit in host memory at once.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

from . import gguf as gg

MAGIC = 0x46554747  # "GGUF" little-endian (types.go:8)
VERSION_MIN, VERSION_MAX = 1, 3
ALIGNMENT = 32      # reader.go:93

# MetaValueType (types.go:18-33)
(T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STRING, T_ARRAY, T_U64, T_I64,
 T_F64) = range(13)
_SCALAR = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i",
           T_F32: "<f", T_BOOL: "<B", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}
MAX_STRING = 1 << 24
MAX_ARRAY = 1 << 20


class GGUFError(ValueError):
    """A malformed or unsupported file (the reference's gguf errors)."""


@dataclass
class MetaValue:
    key: str
    type: int
    value: object  # int / float / bool / str, or ArrayValue


@dataclass
class ArrayValue:
    elem_type: int
    values: list


@dataclass
class TensorInfo:
    """gguf.TensorInfo (types.go:154-160); offset is absolute once read."""
    name: str
    dims: list            # innermost first
    type: int
    offset: int

    def n_elements(self) -> int:  # types.go:162-168
        n = 1
        for d in self.dims:
            n *= int(d)
        return n

    def byte_size(self) -> int:
        return gg.byte_size(self.type, self.n_elements())

    def shape(self) -> list:
        """ggufDimsToShape (flash/storage.go:323-329): outermost first."""
        return [int(d) for d in reversed(self.dims)]

    def row_bytes(self) -> int:
        """Bytes of one row of dims[0] elements (storage.go:277-281)."""
        return gg.byte_size(self.type, int(self.dims[0]))


@dataclass
class GGUFFile:
    """gguf.File (reader.go:11-22)."""
    version: int
    tensor_count: int
    meta_count: int
    meta: dict = field(default_factory=dict)
    tensors: list = field(default_factory=list)
    by_name: dict = field(default_factory=dict)
    data_offset: int = 0
    path: str = ""

    # -- metadata getters (reader.go:121-201) ------------------------------
    def _get(self, key):
        if key not in self.meta:
            raise GGUFError(f"gguf: metadata key {key!r} not found")
        return self.meta[key]

    def meta_string(self, key: str) -> str:
        v = self._get(key)
        if v.type != T_STRING:
            raise GGUFError(f"gguf: metadata key {key!r} is not a string")
        return v.value

    def meta_uint32(self, key: str) -> int:
        v = self._get(key)
        if v.type == T_U32:
            return v.value
        if v.type == T_U64:
            return v.value & 0xFFFFFFFF  # uint32(val)
        if v.type == T_I32:
            return v.value & 0xFFFFFFFF
        raise GGUFError(f"gguf: metadata key {key!r} is not uint32")

    def meta_uint64(self, key: str) -> int:
        v = self._get(key)
        if v.type in (T_U64, T_U32):
            return v.value
        raise GGUFError(f"gguf: metadata key {key!r} is not uint64")

    def meta_float32(self, key: str) -> float:
        v = self._get(key)
        if v.type != T_F32:
            raise GGUFError(f"gguf: metadata key {key!r} is not float32")
        return v.value

    def meta_string_array(self, key: str) -> list:
        v = self._get(key)
        if v.type != T_ARRAY:
            raise GGUFError(f"gguf: metadata key {key!r} is not an array")
        if any(not isinstance(x, str) for x in v.value.values):
            raise GGUFError("gguf: array element is not string")
        return list(v.value.values)

    def meta_int(self, key: str) -> int:
        """Loader.metaInt (model/loader.go:327-341): any of u32/u64/i32/i64."""
        v = self._get(key)
        if v.type in (T_U32, T_U64, T_I32, T_I64):
            return int(v.value)
        raise GGUFError(f"metadata key {key!r} is not an integer")

    # -- tensor data ---------------------------------------------------------
    def tensor_bytes(self, ti: TensorInfo) -> np.ndarray:
        """ReadTensorData (reader.go:205-227) as a read-only memory map (uint8)."""
        n = ti.byte_size()
        size = Path(self.path).stat().st_size
        if ti.offset + n > size:
            raise GGUFError(f"gguf: tensor {ti.name!r} extends past the end of the file")
        return np.memmap(self.path, dtype=np.uint8, mode="r", offset=ti.offset, shape=(n,))

    def tensor_rows(self, name: str) -> np.ndarray:
        """A 2-D tensor's bytes as [rows, row_bytes] (rows = dims[1])."""
        ti = self.by_name.get(name)
        if ti is None:
            raise GGUFError(f"tensor {name!r} not found in GGUF")
        if len(ti.dims) != 2:
            raise GGUFError(f"tensor {name!r} is not 2-D")
        return self.tensor_bytes(ti).reshape(int(ti.dims[1]), ti.row_bytes())


class _Reader:
    def __init__(self, f):
        self.f = f

    def take(self, n: int) -> bytes:
        b = self.f.read(n)
        if len(b) != n:
            raise GGUFError("gguf: unexpected end of file")
        return b

    def scalar(self, t: int):
        fmt = _SCALAR[t]
        v = struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]
        return bool(v) if t == T_BOOL else v

    def string(self) -> str:
        n = self.scalar(T_U64)
        if n > MAX_STRING:
            raise GGUFError(f"gguf: string too long: {n}")
        return self.take(n).decode("utf-8", errors="replace")

    def value(self, t: int):
        if t == T_STRING:
            return self.string()
        if t == T_ARRAY:
            et = self.scalar(T_U32)
            n = self.scalar(T_U64)
            if n > MAX_ARRAY:
                raise GGUFError(f"gguf: array too large: {n}")
            return ArrayValue(et, [self.value(et) for _ in range(n)])
        if t not in _SCALAR:
            raise GGUFError(f"unknown MetaValueType {t}")
        return self.scalar(t)


def open_gguf(path) -> GGUFFile:
    """gguf.Open (reader.go:27-115): metadata and descriptors only."""
    path = str(path)
    with open(path, "rb") as f:
        r = _Reader(f)
        magic = r.scalar(T_U32)
        if magic != MAGIC:
            raise GGUFError(f"gguf: bad magic 0x{magic:08x} (want 0x{MAGIC:08x})")
        version = r.scalar(T_U32)
        if not VERSION_MIN <= version <= VERSION_MAX:
            raise GGUFError(f"gguf: unsupported version {version}")
        n_t, n_kv = r.scalar(T_U64), r.scalar(T_U64)
        gf = GGUFFile(version=version, tensor_count=n_t, meta_count=n_kv, path=path)
        for _ in range(n_kv):
            key = r.string()
            t = r.scalar(T_U32)
            gf.meta[key] = MetaValue(key, t, r.value(t))
        for _ in range(n_t):
            name = r.string()
            nd = r.scalar(T_U32)
            if nd > 4:
                raise GGUFError(f"too many dimensions: {nd}")
            dims = [r.scalar(T_U64) for _ in range(nd)]
            t = r.scalar(T_U32)
            off = r.scalar(T_U64)
            ti = TensorInfo(name, dims, t, off)
            gf.tensors.append(ti)
            gf.by_name[name] = ti
        pos = f.tell()
    gf.data_offset = (pos + ALIGNMENT - 1) // ALIGNMENT * ALIGNMENT
    for ti in gf.tensors:
        ti.offset += gf.data_offset
    return gf


# ---------------------------------------------------------------------------
# Writer
# ---------------------------------------------------------------------------
def _enc_string(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _enc_value(t: int, v) -> bytes:
    if t == T_STRING:
        return _enc_string(v)
    if t == T_ARRAY:
        et, vals = (v.elem_type, v.values) if isinstance(v, ArrayValue) else v
        return struct.pack("<IQ", et, len(vals)) + b"".join(_enc_value(et, x) for x in vals)
    return struct.pack(_SCALAR[t], int(v) if t == T_BOOL else v)


def write_gguf(path, meta, tensors, version: int = 3) -> None:
    """Write a GGUF file.

    meta: iterable of (key, value_type, value) (arrays: (elem_type, [values]));
    tensors: iterable of (name, dims innermost first, ggml_type, data) where
    data is bytes-like of exactly ByteSize(prod(dims)) bytes.
    """
    meta = list(meta)
    tensors = list(tensors)
    head = struct.pack("<IIQQ", MAGIC, version, len(tensors), len(meta))
    head += b"".join(_enc_string(k) + struct.pack("<I", t) + _enc_value(t, v) for k, t, v in meta)
    rel, infos, blobs = 0, [], []
    for name, dims, t, data in tensors:
        buf = np.ascontiguousarray(np.frombuffer(memoryview(data).cast("B"), dtype=np.uint8))
        n = 1
        for d in dims:
            n *= int(d)
        if buf.size != gg.byte_size(t, n):
            raise GGUFError(f"tensor {name!r}: {buf.size} bytes, want {gg.byte_size(t, n)}")
        if len(dims) > 4:
            raise GGUFError(f"too many dimensions: {len(dims)}")
        rel = (rel + ALIGNMENT - 1) // ALIGNMENT * ALIGNMENT
        infos.append(_enc_string(name) + struct.pack("<I", len(dims)) +
                     b"".join(struct.pack("<Q", int(d)) for d in dims) + struct.pack("<IQ", t, rel))
        blobs.append((rel, buf))
        rel += buf.size
    head += b"".join(infos)
    data_off = (len(head) + ALIGNMENT - 1) // ALIGNMENT * ALIGNMENT
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * (data_off - len(head)))
        pos = 0
        for off, buf in blobs:
            f.write(b"\0" * (off - pos))
            f.write(buf.tobytes())
            pos = off + buf.size
