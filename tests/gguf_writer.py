"""Test helper: writes GGUF v2/v3 files byte by byte, including malformed ones.

Layout (GGUF v3): magic "GGUF", u32 version, u64 tensor count, u64 metadata
count, the metadata entries (string key, u32 value type, value), the tensor
directory (string name, u32 n_dims, u64 dims, u32 ggml type, u64 offset
relative to the data section), zero padding to the alignment, then the
payloads.  Strings are u64 length + UTF-8 bytes.  Each directory entry and
metadata entry is kept as its own byte string so a test can corrupt exactly
one field.
"""
from __future__ import annotations

import struct
from collections.abc import Sequence

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
        U64: "<Q", I64: "<q", F64: "<d"}


def s(text: str) -> bytes:
    raw = text.encode()
    return struct.pack("<Q", len(raw)) + raw


def value(vtype: int, v, etype: int | None = None) -> bytes:
    """Encoded value (without the type word, except inside arrays' header)."""
    if vtype == STRING:
        return s(v)
    if vtype == ARRAY:
        return struct.pack("<IQ", etype, len(v)) + b"".join(value(etype, e) for e in v)
    return struct.pack(_FMT[vtype], v)


class Writer:
    def __init__(self, alignment: int | None = 32, architecture: str | None = "qwen3"):
        self.meta: list[bytes] = []
        self.dirs: list[bytes] = []
        self.payloads: list[tuple[int, bytes]] = []  # (relative offset, bytes)
        self.alignment = alignment or 32
        self._next = 0
        if architecture is not None:
            self.kv("general.architecture", STRING, architecture)
        if alignment is not None:
            self.kv("general.alignment", U32, alignment)

    def kv(self, key: str, vtype: int, v, etype: int | None = None) -> None:
        self.meta.append(s(key) + struct.pack("<I", vtype) + value(vtype, v, etype))

    def raw_kv(self, key: str, vtype: int, payload: bytes) -> None:
        self.meta.append(s(key) + struct.pack("<I", vtype) + payload)

    def tensor(self, name: str, dims: Sequence[int], ggml_type: int, payload: bytes,
               offset: int | None = None, name_len: int | None = None, n_dims: int | None = None) -> int:
        """Add a tensor; its payload goes at the next aligned offset unless given."""
        if offset is None:
            offset = self._next
            self._next = -(-(offset + len(payload)) // self.alignment) * self.alignment
        raw = name.encode()
        self.dirs.append(struct.pack("<Q", len(raw) if name_len is None else name_len) + raw
                         + struct.pack("<I", len(dims) if n_dims is None else n_dims)
                         + b"".join(struct.pack("<Q", d) for d in dims)
                         + struct.pack("<I", ggml_type) + struct.pack("<Q", offset))
        self.payloads.append((offset, payload))
        return offset

    def bytes(self, magic: bytes = b"GGUF", version: int = 3, n_tensors: int | None = None,
              n_meta: int | None = None, truncate: int = 0) -> bytes:
        head = (magic + struct.pack("<I", version)
                + struct.pack("<q", len(self.dirs) if n_tensors is None else n_tensors)
                + struct.pack("<q", len(self.meta) if n_meta is None else n_meta)
                + b"".join(self.meta) + b"".join(self.dirs))
        start = -(-len(head) // self.alignment) * self.alignment
        end = max([o + len(p) for o, p in self.payloads], default=0)
        body = bytearray(end)
        for o, p in self.payloads:
            body[o:o + len(p)] = p
        out = head + bytes(start - len(head)) + bytes(body)
        return out[:len(out) - truncate] if truncate else out
