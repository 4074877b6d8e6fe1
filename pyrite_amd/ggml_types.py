"""GGML type geometry for the 21 types the kernels implement.

Same ids, names, block sizes and bytes per block as the reference registry
(pyrite/ggml_types.py:34-74), and the same row-size rule (:117-137).
"""
from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class GGMLTypeSpec:
    type_id: int
    name: str
    block_size: int
    bytes_per_block: int

    @property
    def quantized(self) -> bool:
        return self.block_size > 1


_TYPES = {
    0: GGMLTypeSpec(0, "F32", 1, 4),
    1: GGMLTypeSpec(1, "F16", 1, 2),
    2: GGMLTypeSpec(2, "Q4_0", 32, 18),
    3: GGMLTypeSpec(3, "Q4_1", 32, 20),
    6: GGMLTypeSpec(6, "Q5_0", 32, 22),
    7: GGMLTypeSpec(7, "Q5_1", 32, 24),
    8: GGMLTypeSpec(8, "Q8_0", 32, 34),
    9: GGMLTypeSpec(9, "Q8_1", 32, 36),
    10: GGMLTypeSpec(10, "Q2_K", 256, 84),
    11: GGMLTypeSpec(11, "Q3_K", 256, 110),
    12: GGMLTypeSpec(12, "Q4_K", 256, 144),
    13: GGMLTypeSpec(13, "Q5_K", 256, 176),
    14: GGMLTypeSpec(14, "Q6_K", 256, 210),
    20: GGMLTypeSpec(20, "IQ4_NL", 32, 18),
    23: GGMLTypeSpec(23, "IQ4_XS", 256, 136),
    24: GGMLTypeSpec(24, "I8", 1, 1),
    25: GGMLTypeSpec(25, "I16", 1, 2),
    26: GGMLTypeSpec(26, "I32", 1, 4),
    27: GGMLTypeSpec(27, "I64", 1, 8),
    28: GGMLTypeSpec(28, "F64", 1, 8),
    30: GGMLTypeSpec(30, "BF16", 1, 2),
}

BY_NAME = {t.name: t.type_id for t in _TYPES.values()}


def spec(type_id: int) -> GGMLTypeSpec:
    if not isinstance(type_id, int):
        raise TypeError(f"GGML tensor type must be an integer, got {type_id!r}")
    found = _TYPES.get(type_id)
    if found is None:
        raise ValueError(f"unsupported GGML tensor type: {type_id}")
    return found


def type_name(type_id: int) -> str:
    found = _TYPES.get(type_id)
    return found.name if found else f"UNKNOWN({type_id})"


def row_size(elements: int, type_id: int) -> int:
    """Bytes of one row of ``elements`` values (pyrite/ggml_types.py:117-137)."""
    t = spec(type_id)
    if elements < 0:
        raise ValueError("elements must be non-negative")
    if elements == 0:
        return 0
    if t.block_size != 1 and elements % t.block_size:
        raise ValueError(f"{t.name} row requires element count divisible by {t.block_size}, got {elements}")
    return elements // t.block_size * t.bytes_per_block


def tensor_size(rows: int, cols: int, type_id: int) -> int:
    return rows * row_size(cols, type_id)
