"""Bounds-checked GGUF v2/v3 reader: the tensor directory the HBM loader uploads from.

Mirrors the public surface and error behaviour of the reference reader
(pyrite/adapters/gguf.py:12-389): ``GGUFHeader``, ``GGUFTensor``,
``GGUFError`` (a ``ValueError``), and ``GGUFReader`` with ``header()``,
``metadata()``, ``get()``, ``tensor_index()``, ``tensor()``,
``has_tensor()``, ``tensor_names()``, ``tensor_data_offset``,
``size_bytes`` and ``read_tensor()``, the same safety limits and the same
rejections (bad magic, v1 or > v3, absurd counts, strings longer than what
remains, duplicate keys and names, names of 64+ bytes, more than 4 dims, zero
dims, unknown block types, unaligned, out-of-file or overlapping payloads).

The parse runs over a read-only memory map of the file: every field is
decoded from the mapped bytes with explicit bounds, and arrays of fixed-width
numbers (a 151936-entry token-score table, say) are decoded in one numpy
call instead of element by element.  Parsing is lazy, as in the reference:
nothing is read until an accessor is called.
"""
from __future__ import annotations

import mmap
import struct
from dataclasses import dataclass
from pathlib import Path
from typing import Any

import numpy as np

from .ggml_types import row_size
from .ggml_types import spec as ggml_spec


@dataclass(frozen=True)
class GGUFHeader:
    version: int
    tensor_count: int
    metadata_count: int
    alignment: int
    data_offset: int


@dataclass(frozen=True)
class GGUFTensor:
    """One tensor of the directory; ``offset`` is absolute in the file."""
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
        # unused GGML dimensions are 1, so a 0-dim tensor is one element
        n = 1
        for d in self.dims:
            n *= d
        return n


class GGUFError(ValueError):
    """A GGUF file that cannot be parsed safely; the message names the field."""


# GGUF metadata value types and the numpy dtype of the fixed-width ones.
T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL = 0, 1, 2, 3, 4, 5, 6, 7
T_STRING, T_ARRAY, T_U64, T_I64, T_F64 = 8, 9, 10, 11, 12
_FIXED = {T_U8: "<u1", T_I8: "<i1", T_U16: "<u2", T_I16: "<i2", T_U32: "<u4", T_I32: "<i4",
          T_F32: "<f4", T_U64: "<u8", T_I64: "<i8", T_F64: "<f8"}


class _Reader:
    """Cursor over the mapped file; every read is checked against the end."""

    MAX_STRING_BYTES = 4 * 1024 * 1024

    def __init__(self, buf, limit: int):
        self.buf = buf
        self.pos = 0
        self.limit = limit

    @property
    def remaining(self) -> int:
        return max(0, self.limit - self.pos)

    def take(self, n: int) -> bytes:
        if n < 0:
            raise GGUFError(f"negative GGUF read of {n} bytes")
        if n > self.remaining:
            raise GGUFError(f"truncated GGUF checkpoint: wanted {n} bytes at offset {self.pos}, "
                            f"got {self.remaining}")
        v = self.buf[self.pos:self.pos + n]  # a copy: no view of the map outlives the parse
        self.pos += n
        return v

    def scalar(self, fmt: str):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def u32(self) -> int:
        return self.scalar("<I")

    def u64(self) -> int:
        return self.scalar("<Q")

    def string(self, label: str = "string") -> str:
        n = self.u64()
        if n > self.remaining:
            raise GGUFError(f"GGUF {label} claims {n} bytes but only {self.remaining} remain in the file")
        if n > self.MAX_STRING_BYTES:
            raise GGUFError(f"GGUF {label} length {n} exceeds the {self.MAX_STRING_BYTES}-byte safety limit")
        try:
            return self.take(n).decode("utf-8")
        except UnicodeDecodeError as exc:
            raise GGUFError(f"invalid UTF-8 in GGUF {label}") from exc


class GGUFReader:
    """Bounds-checked, lazy reader of GGUF v2-v3 checkpoints."""

    MAGIC = b"GGUF"
    DEFAULT_ALIGNMENT = 32   # GGUF_DEFAULT_ALIGNMENT
    MAX_DIMS = 4             # GGML_MAX_DIMS
    MAX_NAME = 64            # GGML_MAX_NAME: names must be shorter
    MIN_VERSION = 2          # v1 used 32-bit counts; refused
    MAX_VERSION = 3
    MAX_TENSORS = 10_000_000
    MAX_METADATA = 1_000_000
    MAX_ARRAY = 100_000_000
    MAX_STRING_BYTES = _Reader.MAX_STRING_BYTES

    def __init__(self, path: Path | str):
        self.path = Path(path)
        self._parsed = False
        self._header: GGUFHeader | None = None
        self._metadata: dict[str, Any] = {}
        self._tensors: tuple[GGUFTensor, ...] = ()
        self._index: dict[str, GGUFTensor] = {}
        self._size = 0

    # ------------------------------------------------------------ accessors
    def header(self) -> GGUFHeader:
        self._ensure_parsed()
        return self._header

    def metadata(self) -> dict[str, Any]:
        self._ensure_parsed()
        return dict(self._metadata)

    def get(self, key: str, default: Any = None) -> Any:
        self._ensure_parsed()
        return self._metadata.get(key, default)

    def tensor_index(self) -> tuple[GGUFTensor, ...]:
        self._ensure_parsed()
        return self._tensors

    def tensor(self, name: str) -> GGUFTensor:
        self._ensure_parsed()
        try:
            return self._index[name]
        except KeyError as exc:
            raise KeyError(f"missing GGUF tensor: {name}") from exc

    def has_tensor(self, name: str) -> bool:
        self._ensure_parsed()
        return name in self._index

    def tensor_names(self) -> tuple[str, ...]:
        return tuple(t.name for t in self.tensor_index())

    @property
    def tensor_data_offset(self) -> int:
        self._ensure_parsed()
        return self._header.data_offset

    @property
    def size_bytes(self) -> int:
        self._ensure_parsed()
        return self._size

    def read_tensor(self, tensor: GGUFTensor) -> bytes:
        """The tensor's payload bytes, verbatim."""
        self._ensure_parsed()
        if tensor.offset < 0 or tensor.end > self._size:
            raise ValueError(f"tensor {tensor.name!r} lies outside the checkpoint")
        with self.path.open("rb") as fh:
            fh.seek(tensor.offset)
            data = fh.read(tensor.size)
        if len(data) != tensor.size:
            raise ValueError(f"truncated tensor payload: {tensor.name}")
        return data

    def describe_type(self, ggml_type: int) -> str:
        return ggml_spec(ggml_type).name

    # ---------------------------------------------------------------- parse
    def _ensure_parsed(self) -> None:
        if self._parsed:
            return
        if not self.path.is_file():
            raise FileNotFoundError(self.path)
        size = self.path.stat().st_size
        with self.path.open("rb") as fh:
            if size == 0:
                raise GGUFError(f"not a GGUF checkpoint: {self.path.name} is empty (bad magic)")
            with mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ) as mm:
                self._parse(_Reader(mm, size), size)
        self._parsed = True

    def _parse(self, r: _Reader, size: int) -> None:
        if r.take(4) != self.MAGIC:
            raise GGUFError(f"not a GGUF checkpoint: bad magic in {self.path.name}")
        version = r.u32()
        if version < self.MIN_VERSION:
            raise GGUFError(f"unsupported GGUF version {version}: GGUFv1 used 32-bit counts and is no "
                            "longer supported by the reference implementation; re-export as v3")
        if version > self.MAX_VERSION:
            raise GGUFError(f"unsupported GGUF version {version}: readable versions are "
                            f"v{self.MIN_VERSION}-v{self.MAX_VERSION}")
        n_tensors, n_meta = r.u64(), r.u64()
        if n_tensors > self.MAX_TENSORS or n_meta > self.MAX_METADATA:
            raise GGUFError(f"GGUF header declares {n_tensors} tensors and {n_meta} metadata entries; the "
                            f"safety limits are {self.MAX_TENSORS} and {self.MAX_METADATA}, so the file is "
                            "corrupt or truncated")

        metadata: dict[str, Any] = {}
        alignment = self.DEFAULT_ALIGNMENT
        for _ in range(n_meta):
            key = r.string("metadata key")
            vtype = r.u32()
            if key in metadata:
                raise GGUFError(f"duplicate GGUF metadata key: {key}")
            value = self._value(r, vtype, key)
            metadata[key] = value
            if key == "general.alignment":
                if isinstance(value, bool) or not isinstance(value, int) or value <= 0 or value & (value - 1):
                    raise GGUFError(f"invalid GGUF alignment {value!r}: must be a positive power of two")
                alignment = value

        directory = []
        names: set[str] = set()
        for _ in range(n_tensors):
            name = r.string("tensor name")
            n_dims = r.u32()
            if name in names:
                raise GGUFError(f"duplicate GGUF tensor name: {name}")
            if len(name) >= self.MAX_NAME:
                raise GGUFError(f"tensor name {name[:32]!r}... is {len(name)} bytes; GGML_MAX_NAME is "
                                f"{self.MAX_NAME}")
            names.add(name)
            if n_dims > self.MAX_DIMS:
                raise GGUFError(f"GGUF tensor {name!r} has {n_dims} dimensions; GGML_MAX_DIMS is {self.MAX_DIMS}")
            dims = tuple(int(d) for d in np.frombuffer(r.take(8 * n_dims), dtype="<u8"))
            if any(d == 0 for d in dims):
                raise GGUFError(f"GGUF tensor {name!r} has a zero-sized dimension: {dims}")
            gtype = r.u32()
            rel = r.u64()
            directory.append((name, dims, gtype, rel))

        # tensor data begins at the next multiple of the alignment
        data_offset = -(-r.pos // alignment) * alignment if n_tensors else r.pos
        if data_offset > size:
            raise GGUFError(f"GGUF tensor data starts at {data_offset}, beyond the {size}-byte file")
        tensors = []
        for name, dims, gtype, rel in directory:
            if rel % alignment:
                raise GGUFError(f"unaligned GGUF tensor offset: {name} starts at {rel}, which is not a multiple "
                                f"of the {alignment}-byte alignment")
            try:
                nbytes = self._tensor_size(dims, gtype, name)
            except ValueError as exc:
                raise GGUFError(str(exc)) from exc
            if rel > size - data_offset:
                raise GGUFError(f"GGUF tensor {name} offset {rel} lies beyond the file")
            start = data_offset + rel
            if nbytes > size - start:
                raise GGUFError(f"GGUF tensor {name} needs {nbytes} bytes at {start} but the file ends at {size}")
            tensors.append(GGUFTensor(name, dims, gtype, start, nbytes))
        # payloads may appear in any order but must not overlap
        last_end, last_name = data_offset, ""
        for t in sorted(tensors, key=lambda t: (t.offset, t.end, t.name)):
            if t.offset < last_end:
                raise GGUFError(f"GGUF tensor payload overlaps another tensor: {last_name}, {t.name}")
            last_end, last_name = t.end, t.name

        self._header = GGUFHeader(version, n_tensors, n_meta, alignment, data_offset)
        self._metadata = metadata
        self._tensors = tuple(tensors)
        self._index = {t.name: t for t in tensors}
        self._size = size

    def _value(self, r: _Reader, vtype: int, key: str) -> Any:
        if vtype in _FIXED:
            dt = np.dtype(_FIXED[vtype])
            v = np.frombuffer(r.take(dt.itemsize), dtype=dt)[0]
            return float(v) if dt.kind == "f" else int(v)
        if vtype == T_BOOL:
            b = r.scalar("<B")
            if b not in (0, 1):
                raise GGUFError(f"invalid GGUF boolean value: {b}")
            return bool(b)
        if vtype == T_STRING:
            return r.string(f"metadata value for {key!r}")
        if vtype == T_ARRAY:
            etype, count = r.u32(), r.u64()
            if count > self.MAX_ARRAY:
                raise GGUFError(f"GGUF metadata array {key!r} declares {count} elements, above the "
                                f"{self.MAX_ARRAY} safety limit")
            # every element takes at least one byte: a larger count cannot be real
            if count > r.remaining:
                raise GGUFError(f"GGUF metadata array {key!r} declares {count} elements but only "
                                f"{r.remaining} bytes remain in the file")
            if etype in _FIXED:
                dt = np.dtype(_FIXED[etype])
                arr = np.frombuffer(r.take(count * dt.itemsize), dtype=dt)
                return tuple(arr.tolist())
            if etype == T_BOOL:
                raw = np.frombuffer(r.take(count), dtype=np.uint8)
                bad = raw[raw > 1]
                if bad.size:
                    raise GGUFError(f"invalid GGUF boolean value: {int(bad[0])}")
                return tuple(bool(b) for b in raw)
            return tuple(self._value(r, etype, key) for _ in range(count))
        raise GGUFError(f"unsupported GGUF metadata value type {vtype} for key {key!r}")

    @staticmethod
    def _tensor_size(dims: tuple[int, ...], ggml_type: int, name: str = "") -> int:
        """Payload bytes: rows of dims[0] elements times the product of the other dims."""
        if not dims:
            return row_size(1, ggml_type)
        rows = 1
        for d in dims[1:]:
            rows *= d
        try:
            return row_size(dims[0], ggml_type) * rows
        except (TypeError, ValueError) as exc:
            label = f"tensor {name!r}: " if name else ""
            raise ValueError(f"{label}{exc}") from exc
