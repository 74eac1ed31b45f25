"""GGUF parser: header, KV metadata and tensor table.

Mirrors ``parseGGUF`` of the reference (``webgpu/src/model/gguf.ts:241-299``)
over the same caller-supplied range reader ``read_range(start, end) -> bytes``,
so a file, a memory map or a byte string can back it.  Only header bytes are
read; tensor data is not touched.

Format (little-endian), as the reference documents it (``gguf.ts:1-20``)::

    magic u32 'GGUF' | version u32 (2 or 3) | tensor_count u64 | kv_count u64
    kv_count x { key: string, value_type: u32, value }
    tensor_count x { name: string, n_dims: u32, ne[n_dims]: u64, ggml_type: u32, offset: u64 }
    <padding to general.alignment (default 32)>
    tensor data (offsets relative to the data section start)

Behaviour kept from the reference:
* the header is fetched 4 MiB first and the buffer doubles on demand, capped
  at 512 MiB (``HeaderCursor.ensure``, ``gguf.ts:128-150``);
* ``u64`` / ``i64`` values beyond 2^53 raise, as the reference's Number
  conversion does (``gguf.ts:163-180``);
* tensors have at most 4 dims; ``byte_length`` comes from
  ``ggml_tensor_bytes`` (``gguf.ts:82-92``) and raises on an unknown type or
  an ``ne[0]`` that is not a multiple of the block size;
* ``data_offset = ceil(header_bytes / alignment) * alignment``.

Error texts are the reference's, raised as ``ValueError`` (the reference
throws ``Error``) or ``GGMLTypeError`` for unknown tensor types.
"""

from __future__ import annotations

import dataclasses
import mmap
import os
import struct
from typing import Any, Callable, Dict, List, Optional

from .ggml import GGMLTypeError, ggml_tensor_bytes, ggml_type_traits

__all__ = [
    "GGUF_MAGIC", "GGUFValueType", "GGUFTensorInfo", "GGUFFile", "RangeReader",
    "parse_gguf", "parse_gguf_path", "file_range_reader", "gguf_architecture", "arch_kv",
    "map_tensor_bytes", "gguf_header_bytes", "write_gguf",
]

GGUF_MAGIC = 0x46554747               # 'GGUF' little-endian, gguf.ts:113
INITIAL_FETCH = 4 * 1024 * 1024       # gguf.ts:114
MAX_HEADER = 512 * 1024 * 1024        # gguf.ts:115
_MAX_SAFE = (1 << 53) - 1             # Number.MAX_SAFE_INTEGER

RangeReader = Callable[[int, int], bytes]


class GGUFValueType:
    """KV value type ids (gguf.ts:189-192)."""
    UINT8, INT8, UINT16, INT16, UINT32, INT32 = 0, 1, 2, 3, 4, 5
    FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = 6, 7, 8, 9, 10, 11, 12


@dataclasses.dataclass
class GGUFTensorInfo:
    """One tensor-table entry (``GGUFTensorInfo``, gguf.ts:96-109)."""
    name: str
    ne: List[int]          # GGUF dims, innermost first (ne[0] = contiguous axis)
    shape: List[int]       # reversed ne: [out, in] for matrices
    ggml_type: int
    type_name: str
    offset: int            # absolute byte offset of the data in the file
    byte_length: int
    element_count: int


@dataclasses.dataclass
class GGUFFile:
    """Parsed header (``GGUFFile``, gguf.ts:111-123)."""
    version: int
    tensor_count: int
    kv: Dict[str, Any]
    tensors: Dict[str, GGUFTensorInfo]
    data_offset: int
    alignment: int
    header_bytes: int


class _HeaderCursor:
    """Cursor over progressively fetched header bytes (gguf.ts:119-187)."""

    def __init__(self, read_range: RangeReader, initial: bytes):
        self._read = read_range
        self._buf = bytearray(initial)
        self.pos = 0

    def _ensure(self, n: int) -> None:
        if self.pos + n <= len(self._buf):
            return
        new_len = max(len(self._buf), 1)
        while new_len < self.pos + n:
            new_len *= 2
        if new_len > MAX_HEADER:
            raise ValueError(f"[GGUF] Header exceeds {MAX_HEADER} bytes — corrupt file?")
        more = self._read(len(self._buf), new_len)
        self._buf += more
        if len(self._buf) < self.pos + n:
            raise ValueError(f"[GGUF] Short read growing header buffer: have {len(self._buf)}, "
                             f"need {self.pos + n}")

    def _unpack(self, fmt: str, size: int):
        self._ensure(size)
        v = struct.unpack_from(fmt, self._buf, self.pos)[0]
        self.pos += size
        return v

    def u8(self) -> int: return self._unpack("<B", 1)
    def i8(self) -> int: return self._unpack("<b", 1)
    def u16(self) -> int: return self._unpack("<H", 2)
    def i16(self) -> int: return self._unpack("<h", 2)
    def u32(self) -> int: return self._unpack("<I", 4)
    def i32(self) -> int: return self._unpack("<i", 4)
    def f32(self) -> float: return self._unpack("<f", 4)
    def f64(self) -> float: return self._unpack("<d", 8)

    def u64(self) -> int:
        v = self._unpack("<Q", 8)
        if v > _MAX_SAFE:
            raise ValueError(f"[GGUF] u64 {v} exceeds safe integer")
        return v

    def i64(self) -> int:
        v = self._unpack("<q", 8)
        if v > _MAX_SAFE or v < -_MAX_SAFE:
            raise ValueError(f"[GGUF] i64 {v} exceeds safe integer")
        return v

    def str(self) -> str:
        n = self.u64()
        self._ensure(n)
        s = bytes(self._buf[self.pos:self.pos + n]).decode("utf-8", errors="replace")
        self.pos += n
        return s


def _read_value(c: _HeaderCursor, vtype: int):
    """One KV value of type ``vtype`` (readValue, gguf.ts:194-216)."""
    t = GGUFValueType
    if vtype == t.UINT8: return c.u8()
    if vtype == t.INT8: return c.i8()
    if vtype == t.UINT16: return c.u16()
    if vtype == t.INT16: return c.i16()
    if vtype == t.UINT32: return c.u32()
    if vtype == t.INT32: return c.i32()
    if vtype == t.FLOAT32: return c.f32()
    if vtype == t.BOOL: return c.u8() != 0
    if vtype == t.STRING: return c.str()
    if vtype == t.UINT64: return c.u64()
    if vtype == t.INT64: return c.i64()
    if vtype == t.FLOAT64: return c.f64()
    if vtype == t.ARRAY:
        et = c.u32()
        count = c.u64()
        return [_read_value(c, et) for _ in range(count)]
    raise ValueError(f"[GGUF] Unknown KV value type {vtype}")


def parse_gguf(read_range: RangeReader) -> GGUFFile:
    """Parse header, KV metadata and tensor table (parseGGUF, gguf.ts:241-299)."""
    c = _HeaderCursor(read_range, read_range(0, INITIAL_FETCH))
    magic = c.u32()
    if magic != GGUF_MAGIC:
        raise ValueError(f"[GGUF] Bad magic 0x{magic:x} — not a GGUF file")
    version = c.u32()
    if version < 2 or version > 3:
        raise ValueError(f"[GGUF] Unsupported version {version} (need 2 or 3)")
    tensor_count = c.u64()
    kv_count = c.u64()

    kv: Dict[str, Any] = {}
    for _ in range(kv_count):
        key = c.str()
        vtype = c.u32()
        kv[key] = _read_value(c, vtype)

    alignment = int(kv.get("general.alignment", 32))

    raw = []
    for _ in range(tensor_count):
        name = c.str()
        n_dims = c.u32()
        if n_dims > 4:
            raise ValueError(f'[GGUF] Tensor "{name}" has {n_dims} dims (max 4)')
        ne = [c.u64() for _ in range(n_dims)]
        ggml_type = c.u32()
        rel = c.u64()
        raw.append((name, ne, ggml_type, rel))

    header_bytes = c.pos
    data_offset = -(-header_bytes // alignment) * alignment

    tensors: Dict[str, GGUFTensorInfo] = {}
    for name, ne, ggml_type, rel in raw:
        nbytes = ggml_tensor_bytes(ggml_type, ne)
        count = 1
        for d in ne:
            count *= d
        tensors[name] = GGUFTensorInfo(
            name=name, ne=ne, shape=list(reversed(ne)), ggml_type=ggml_type,
            type_name=ggml_type_traits(ggml_type)[2], offset=data_offset + rel,
            byte_length=nbytes, element_count=count)
    return GGUFFile(version, tensor_count, kv, tensors, data_offset, alignment, header_bytes)


def file_range_reader(path: str) -> RangeReader:
    """A range reader over a local file (short reads at the end, like a File slice)."""
    def read(start: int, end: int) -> bytes:
        with open(path, "rb") as f:
            f.seek(start)
            return f.read(max(0, end - start))
    return read


def parse_gguf_path(path: str) -> GGUFFile:
    return parse_gguf(file_range_reader(path))


def gguf_architecture(file: GGUFFile) -> str:
    """``general.architecture`` (ggufArchitecture, gguf.ts:304-308)."""
    arch = file.kv.get("general.architecture")
    if not isinstance(arch, str):
        raise ValueError("[GGUF] Missing general.architecture")
    return arch


_MISSING = object()


def arch_kv(file: GGUFFile, key: str, fallback: Any = _MISSING) -> Any:
    """``<arch>.<key>`` with an optional fallback (archKV, gguf.ts:311-319)."""
    arch = gguf_architecture(file)
    v = file.kv.get(f"{arch}.{key}")
    if v is None:
        if fallback is not _MISSING:
            return fallback
        raise ValueError(f"[GGUF] Missing KV {arch}.{key}")
    return v


def map_tensor_bytes(path: str, info: GGUFTensorInfo) -> memoryview:
    """Read-only view of one tensor's raw bytes in a memory map of ``path``.

    Raises if the file is shorter than the tensor table says (the reference's
    byte-count assertion on every fetched chunk, gguf-loader.ts:126-140)."""
    size = os.path.getsize(path)
    if info.offset + info.byte_length > size:
        raise ValueError(f"[GGUF] tensor {info.name}: bytes [{info.offset}, "
                         f"{info.offset + info.byte_length}) past end of file ({size} B)")
    with open(path, "rb") as f:
        mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
    return memoryview(mm)[info.offset:info.offset + info.byte_length]


# ---------------------------------------------------------------------------
# Writer (the inverse of parse_gguf): for exporting quantized weights and for
# building model files.  The reference only reads GGUF; its files come from
# llama.cpp's converter.  Layout follows the format above: tensors in the
# order given, each at a multiple of ``alignment`` from the data section start.
# ---------------------------------------------------------------------------

def _infer_vtype(v) -> int:
    t = GGUFValueType
    if isinstance(v, bool):
        return t.BOOL
    if isinstance(v, int):
        return t.UINT32 if 0 <= v < (1 << 32) else t.INT64
    if isinstance(v, float):
        return t.FLOAT32
    if isinstance(v, str):
        return t.STRING
    if isinstance(v, (list, tuple)):
        return t.ARRAY
    raise TypeError(f"no GGUF value type for {type(v).__name__}")


_SCALAR_FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 10: "<Q",
               11: "<q", 12: "<d"}


def _pack_str(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _pack_value(v, vtype: int, elem_type: Optional[int] = None) -> bytes:
    t = GGUFValueType
    if vtype == t.BOOL:
        return struct.pack("<B", 1 if v else 0)
    if vtype == t.STRING:
        return _pack_str(v)
    if vtype == t.ARRAY:
        et = elem_type if elem_type is not None else (_infer_vtype(v[0]) if len(v) else t.UINT32)
        return (struct.pack("<IQ", et, len(v))
                + b"".join(_pack_value(e, et) for e in v))
    if vtype in _SCALAR_FMT:
        return struct.pack(_SCALAR_FMT[vtype], v)
    raise ValueError(f"[GGUF] Unknown KV value type {vtype}")


def gguf_header_bytes(kv: Dict[str, Any], tensors, alignment: int = 32, version: int = 3,
                      kv_types: Optional[Dict[str, Any]] = None) -> tuple:
    """Header bytes (magic .. tensor table) and each tensor's relative offset.

    ``tensors``: sequence of ``(name, ne, ggml_type, nbytes)``.  ``kv_types``
    maps a key to a value type id, or to ``(ARRAY, elem_type)`` for arrays;
    other keys get a type inferred from the Python value."""
    kv = dict(kv)
    if alignment != 32:
        kv.setdefault("general.alignment", alignment)
    kv_types = dict(kv_types or {})
    if "general.alignment" in kv:
        kv_types.setdefault("general.alignment", GGUFValueType.UINT32)
    out = [struct.pack("<IIQQ", GGUF_MAGIC, version, len(tensors), len(kv))]
    for key, v in kv.items():
        spec = kv_types.get(key, _infer_vtype(v))
        vtype, et = (spec if isinstance(spec, tuple) else (spec, None))
        out.append(_pack_str(key) + struct.pack("<I", vtype) + _pack_value(v, vtype, et))
    rel, offsets = 0, []
    for name, ne, ggml_type, nbytes in tensors:
        offsets.append(rel)
        out.append(_pack_str(name) + struct.pack("<I", len(ne))
                   + b"".join(struct.pack("<Q", int(d)) for d in ne)
                   + struct.pack("<IQ", ggml_type, rel))
        rel += -(-int(nbytes) // alignment) * alignment
    return b"".join(out), offsets


def write_gguf(path: str, kv: Dict[str, Any], tensors, alignment: int = 32, version: int = 3,
               kv_types: Optional[Dict[str, Any]] = None) -> None:
    """Write a GGUF file.  ``tensors``: sequence of ``(name, ne, ggml_type, data)``
    with ``data`` the raw GGUF bytes (bytes-like or a numpy array); the byte
    count must equal ``ggml_tensor_bytes(ggml_type, ne)``."""
    import numpy as np

    entries = []
    for name, ne, ggml_type, data in tensors:
        buf = memoryview(np.ascontiguousarray(data).view(np.uint8).reshape(-1)
                         if isinstance(data, np.ndarray) else data).cast("B")
        want = ggml_tensor_bytes(ggml_type, ne)
        if buf.nbytes != want:
            raise ValueError(f"[GGUF] tensor {name}: {buf.nbytes} bytes, type {ggml_type} "
                             f"with ne={list(ne)} needs {want}")
        entries.append((name, list(ne), int(ggml_type), buf))
    header, offsets = gguf_header_bytes(kv, [(n, ne, t, b.nbytes) for n, ne, t, b in entries],
                                        alignment, version, kv_types)
    data_offset = -(-len(header) // alignment) * alignment
    with open(path, "wb") as f:
        f.write(header)
        f.write(b"\0" * (data_offset - len(header)))
        pos = 0
        for (name, ne, t, buf), rel in zip(entries, offsets):
            f.write(b"\0" * (rel - pos))
            f.write(buf)
            pos = rel + buf.nbytes
