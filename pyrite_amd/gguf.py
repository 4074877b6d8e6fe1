"""GGUF v2/v3 tensor directory for the HBM loader.

Interface (kept so code written against the reference reader,
pyrite/adapters/gguf.py, works unchanged): the dataclasses ``GGUFHeader`` and
``GGUFTensor``, the exception ``GGUFError`` (a ``ValueError``), and
``GGUFReader`` with ``header()``, ``metadata()``, ``get()``,
``tensor_index()``, ``tensor()``, ``has_tensor()``, ``tensor_names()``,
``tensor_data_offset``, ``size_bytes``, ``read_tensor()`` and the class limits
``MAX_DIMS``, ``MAX_NAME``, ``MIN_VERSION``/``MAX_VERSION``, ``MAX_TENSORS``,
``MAX_METADATA``, ``MAX_ARRAY``, ``MAX_STRING_BYTES`` and
``DEFAULT_ALIGNMENT``.  Files are parsed lazily, on the first accessor call.

The file format (little-endian throughout):

    "GGUF"  u32 version  u64 n_tensors  u64 n_kv
    n_kv    x  { string key, u32 value type, value }
    n_tensors x { string name, u32 n_dims, u64 dims[n_dims], u32 ggml type,
                  u64 offset relative to the data section }
    zero padding to the alignment (general.alignment, default 32)
    tensor payloads

with string = u64 byte length + UTF-8 bytes and array = u32 element type +
u64 count + elements.  Version 1 used 32-bit counts and is not read.

Parsing happens in two passes over a read-only memory map.  The first decodes
the header, the key/value pairs and the directory records through ``_Span``,
which refuses any read past the end of the file.  The second places the
payloads: it computes each tensor's size from its GGML geometry, then checks
alignment, extent and that no two payloads share a byte.  Fixed-width arrays,
such as a 151936-entry token-score table, are decoded with one numpy call.
"""
from __future__ import annotations

import mmap
import os
import struct
from dataclasses import dataclass
from pathlib import Path
from typing import Any, NamedTuple

import numpy as np

from .ggml_types import row_size


@dataclass(frozen=True)
class GGUFHeader:
    version: int
    tensor_count: int
    metadata_count: int
    alignment: int
    data_offset: int


@dataclass(frozen=True)
class GGUFTensor:
    """A directory entry; ``offset`` is absolute in the file, ``size`` in bytes."""
    name: str
    dims: tuple[int, ...]
    ggml_type: int
    offset: int
    size: int

    @property
    def end(self) -> int:
        return self.offset + self.size

    @property
    def element_count(self) -> int:
        return int(np.prod(self.dims, dtype=object)) if self.dims else 1


class GGUFError(ValueError):
    """The file is not a GGUF checkpoint this reader can use; the message says why."""


# Metadata value types: id -> (struct format, numpy dtype) for fixed-width ones.
_U8, _I8, _U16, _I16, _U32, _I32, _F32, _BOOL, _STRING, _ARRAY, _U64, _I64, _F64 = range(13)
_SCALARS: dict[int, tuple[str, str]] = {
    _U8: ("<B", "<u1"), _I8: ("<b", "<i1"), _U16: ("<H", "<u2"), _I16: ("<h", "<i2"),
    _U32: ("<I", "<u4"), _I32: ("<i", "<i4"), _F32: ("<f", "<f4"), _U64: ("<Q", "<u8"),
    _I64: ("<q", "<i8"), _F64: ("<d", "<f8"),
}


class _Span:
    """Decoding position over the mapped bytes [0, end)."""

    def __init__(self, mv: memoryview, end: int, string_cap: int):
        self.mv = mv
        self.at = 0
        self.end = end
        self.string_cap = string_cap

    def left(self) -> int:
        return self.end - self.at

    def bytes(self, n: int, what: str) -> bytes:
        if n > self.left():
            raise GGUFError(f"file ends at byte {self.end}: {what} needs {n} bytes from offset {self.at}")
        out = bytes(self.mv[self.at:self.at + n])
        self.at += n
        return out

    def scalar(self, fmt: str, what: str):
        return struct.unpack(fmt, self.bytes(struct.calcsize(fmt), what))[0]

    def text(self, what: str) -> str:
        start = self.at
        n = self.scalar("<Q", f"the length of {what}")
        if n > self.left():
            raise GGUFError(f"{what} at offset {start} declares {n} bytes; only {self.left()} are left")
        if n > self.string_cap:
            raise GGUFError(f"{what} at offset {start} declares {n} bytes, over the {self.string_cap}-byte "
                            "cap on strings")
        raw = self.bytes(n, what)
        try:
            return raw.decode("utf-8")
        except UnicodeDecodeError as exc:
            raise GGUFError(f"{what} at offset {start} is not UTF-8") from exc


class _Record(NamedTuple):
    """A directory entry before its payload is placed."""
    name: str
    dims: tuple[int, ...]
    ggml_type: int
    rel: int


class GGUFReader:
    """Lazy, bounds-checked reader of GGUF v2 and v3 checkpoints."""

    MAGIC = b"GGUF"
    DEFAULT_ALIGNMENT = 32   # GGUF_DEFAULT_ALIGNMENT
    MAX_DIMS = 4             # GGML_MAX_DIMS
    MAX_NAME = 64            # GGML_MAX_NAME (a name must be shorter)
    MIN_VERSION = 2
    MAX_VERSION = 3
    MAX_TENSORS = 10_000_000
    MAX_METADATA = 1_000_000
    MAX_ARRAY = 100_000_000
    MAX_STRING_BYTES = 4 << 20

    def __init__(self, path: Path | str):
        self.path = Path(path)
        self._state: tuple[GGUFHeader, dict[str, Any], tuple[GGUFTensor, ...], int] | None = None
        self._by_name: dict[str, GGUFTensor] = {}

    # ---------------------------------------------------------------- access
    def _loaded(self):
        if self._state is None:
            self._state = self._load()
            self._by_name = {t.name: t for t in self._state[2]}
        return self._state

    def header(self) -> GGUFHeader:
        return self._loaded()[0]

    def metadata(self) -> dict[str, Any]:
        return dict(self._loaded()[1])

    def get(self, key: str, default: Any = None) -> Any:
        return self._loaded()[1].get(key, default)

    def tensor_index(self) -> tuple[GGUFTensor, ...]:
        return self._loaded()[2]

    def tensor(self, name: str) -> GGUFTensor:
        self._loaded()
        found = self._by_name.get(name)
        if found is None:
            raise KeyError(f"no tensor named {name!r} in {self.path.name}")
        return found

    def has_tensor(self, name: str) -> bool:
        self._loaded()
        return name in self._by_name

    def tensor_names(self) -> tuple[str, ...]:
        return tuple(t.name for t in self._loaded()[2])

    @property
    def tensor_data_offset(self) -> int:
        return self._loaded()[0].data_offset

    @property
    def size_bytes(self) -> int:
        return self._loaded()[3]

    def read_tensor(self, tensor: GGUFTensor) -> bytes:
        """The payload bytes of ``tensor`` as stored (one positioned read)."""
        size = self._loaded()[3]
        if tensor.offset < 0 or tensor.size < 0 or tensor.end > size:
            raise ValueError(f"{tensor.name!r} spans bytes [{tensor.offset}, {tensor.end}) of a {size}-byte file")
        fd = os.open(self.path, os.O_RDONLY)
        try:
            data = os.pread(fd, tensor.size, tensor.offset)
        finally:
            os.close(fd)
        if len(data) != tensor.size:
            raise ValueError(f"{tensor.name!r}: read {len(data)} of {tensor.size} payload bytes")
        return data

    # ----------------------------------------------------------------- parse
    def _load(self):
        if not self.path.is_file():
            raise FileNotFoundError(self.path)
        size = self.path.stat().st_size
        if size < 4:
            raise GGUFError(f"{self.path.name} has {size} bytes: too short for the GGUF magic")
        with self.path.open("rb") as fh, mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ) as mm:
            mv = memoryview(mm)
            try:
                version, kv, records, end_of_directory = self._decode(_Span(mv, size, self.MAX_STRING_BYTES))
            finally:
                mv.release()
        alignment = self._alignment(kv)
        data_offset = end_of_directory if not records else -(-end_of_directory // alignment) * alignment
        if data_offset > size:
            raise GGUFError(f"the data section would start at byte {data_offset}, past the end of the "
                            f"{size}-byte file")
        tensors = self._place(records, alignment, data_offset, size)
        header = GGUFHeader(version, len(records), len(kv), alignment, data_offset)
        return header, kv, tensors, size

    def _decode(self, sp: _Span):
        magic = sp.bytes(4, "the magic")
        if magic != self.MAGIC:
            raise GGUFError(f"{self.path.name}: first four bytes are {magic!r}, not the GGUF magic")
        version = sp.scalar("<I", "the version")
        if not self.MIN_VERSION <= version <= self.MAX_VERSION:
            raise GGUFError(f"GGUF version {version} is not readable here (versions {self.MIN_VERSION} to "
                            f"{self.MAX_VERSION} are; version 1 used 32-bit counts)")
        n_tensors = sp.scalar("<Q", "the tensor count")
        n_kv = sp.scalar("<Q", "the key/value count")
        if n_tensors > self.MAX_TENSORS or n_kv > self.MAX_METADATA:
            raise GGUFError(f"the header counts ({n_tensors} tensors, {n_kv} key/value pairs) exceed the "
                            f"safety limits ({self.MAX_TENSORS}, {self.MAX_METADATA})")
        kv: dict[str, Any] = {}
        for i in range(n_kv):
            key = sp.text(f"metadata key {i}")
            if key in kv:
                raise GGUFError(f"key {key!r} appears twice in the metadata")
            vtype = sp.scalar("<I", f"the value type of {key!r}")
            kv[key] = self._value(sp, vtype, key)
        records: list[_Record] = []
        seen: set[str] = set()
        for i in range(n_tensors):
            name = sp.text(f"tensor name {i}")
            if len(name.encode()) >= self.MAX_NAME:
                raise GGUFError(f"tensor name of {len(name.encode())} bytes ({name[:24]!r}...) is not shorter "
                                f"than GGML_MAX_NAME = {self.MAX_NAME}")
            if name in seen:
                raise GGUFError(f"tensor {name!r} appears twice in the directory")
            seen.add(name)
            n_dims = sp.scalar("<I", f"the rank of {name!r}")
            if n_dims > self.MAX_DIMS:
                raise GGUFError(f"tensor {name!r} has {n_dims} dimensions; GGML allows at most {self.MAX_DIMS}")
            dims = tuple(int(d) for d in np.frombuffer(sp.bytes(8 * n_dims, f"the shape of {name!r}"), "<u8"))
            if 0 in dims:
                raise GGUFError(f"tensor {name!r} has an empty dimension in {dims}")
            gtype = sp.scalar("<I", f"the type of {name!r}")
            rel = sp.scalar("<Q", f"the offset of {name!r}")
            records.append(_Record(name, dims, gtype, rel))
        return version, kv, records, sp.at

    def _value(self, sp: _Span, vtype: int, key: str) -> Any:
        if vtype in _SCALARS:
            v = sp.scalar(_SCALARS[vtype][0], f"the value of {key!r}")
            return float(v) if isinstance(v, float) else int(v)
        if vtype == _BOOL:
            return self._bools(sp.bytes(1, f"the value of {key!r}"))[0]
        if vtype == _STRING:
            return sp.text(f"the value of {key!r}")
        if vtype == _ARRAY:
            etype = sp.scalar("<I", f"the element type of {key!r}")
            count = sp.scalar("<Q", f"the element count of {key!r}")
            if count > self.MAX_ARRAY:
                raise GGUFError(f"array {key!r} declares {count} elements, over the {self.MAX_ARRAY}-element cap")
            if count > sp.left():  # every element takes at least one byte
                raise GGUFError(f"array {key!r} declares {count} elements; only {sp.left()} bytes are left")
            if etype in _SCALARS:
                dt = np.dtype(_SCALARS[etype][1])
                return tuple(np.frombuffer(sp.bytes(count * dt.itemsize, f"the elements of {key!r}"), dt).tolist())
            if etype == _BOOL:
                return self._bools(sp.bytes(count, f"the elements of {key!r}"))
            return tuple(self._value(sp, etype, key) for _ in range(count))
        raise GGUFError(f"key {key!r} has value type {vtype}, which GGUF does not define")

    @staticmethod
    def _bools(raw: bytes) -> tuple[bool, ...]:
        arr = np.frombuffer(raw, np.uint8)
        if (arr > 1).any():
            raise GGUFError(f"boolean value byte {int(arr[arr > 1][0])} is neither 0 nor 1")
        return tuple(bool(b) for b in arr)

    def _alignment(self, kv: dict[str, Any]) -> int:
        a = kv.get("general.alignment", self.DEFAULT_ALIGNMENT)
        if isinstance(a, bool) or not isinstance(a, int) or a <= 0 or a & (a - 1):
            raise GGUFError(f"general.alignment = {a!r} is not a positive power of two")
        return a

    @staticmethod
    def _place(records: list[_Record], alignment: int, data_offset: int, size: int) -> tuple[GGUFTensor, ...]:
        room = size - data_offset
        placed = []
        for r in records:
            if r.rel % alignment:
                raise GGUFError(f"tensor {r.name!r}: payload offset {r.rel} is not a multiple of the "
                                f"{alignment}-byte alignment")
            # bytes = rows of dims[0] elements x the other dims (a 0-D tensor is one element)
            try:
                nbytes = row_size(r.dims[0] if r.dims else 1, r.ggml_type)
            except (TypeError, ValueError) as exc:
                raise GGUFError(f"tensor {r.name!r}: {exc}") from exc
            for d in r.dims[1:]:
                nbytes *= d
            if r.rel > room:
                raise GGUFError(f"tensor {r.name!r}: payload offset {r.rel} is past the end of the data section")
            if nbytes > room - r.rel:
                raise GGUFError(f"tensor {r.name!r}: {nbytes} payload bytes from byte {data_offset + r.rel} run "
                                f"past the end of the file ({size} bytes)")
            placed.append(GGUFTensor(r.name, r.dims, r.ggml_type, data_offset + r.rel, nbytes))
        # payloads may be stored in any order, but no byte may belong to two tensors
        by_start = sorted(placed, key=lambda t: (t.offset, t.end))
        for a, b in zip(by_start, by_start[1:]):
            if b.offset < a.end:
                raise GGUFError(f"payloads of tensors {a.name!r} and {b.name!r} overlap")
        return tuple(placed)
