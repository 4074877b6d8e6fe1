"""Write the golden fixtures under tests/golden/ (run in the build container only).

Two sources, both read from the reference checkout at /root/reference:

1. ``oracle/_ref/libpyrite_ref.so`` -- the reference's pyrite/kernels/native.c
   compiled unmodified by oracle/Makefile.  For every one of the 21 types it
   produces the matvec and dequantize outputs on
   (a) the payload recipe of tests/test_native_kernels.py:61-91 (LCG bytes,
       seed 20240607, finite fp16 scale words, x = cos(0.13 i) * 0.4),
   (b) seeded random bytes (numpy PCG64) with non-finite half words replaced,
   (c) blocks whose fp16 scale words walk through special values (zero, signed
       zero, smallest/largest subnormal, smallest normal, largest finite,
       negative scales).
2. tests/k_quant.py of the reference, imported here to record its encoder
   outputs byte for byte; nothing else pins the quantizer bytes.  Inputs are
   the weights of tests/test_native_kernels.py:136-139 and seeded N(0, 0.02)
   values.

Payloads and outputs are stored in .npz files (no pickles).  The fixtures are
data only; this script is not imported by any test.
"""
from __future__ import annotations

import hashlib
import importlib.util
import math
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle.oracle import TYPES, lcg_payload, oracle, reference  # noqa: E402
from tests.gpu_util import HALF_WORDS, random_payload  # noqa: E402

OUT = Path(__file__).resolve().parent
REFERENCE_TESTS = Path("/root/reference/tests")

# fp16 words walked through by the special-scale payloads
SPECIAL_HALVES = [0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x7BFF, 0xBC00, 0x3C00,
                  0x0200, 0x8001, 0xFBFF, 0x1400, 0x2E66, 0xB555]

def ref_vector(cols: int) -> np.ndarray:
    return np.array([math.cos(i * 0.13) * 0.4 for i in range(cols)], dtype=np.float64)


def special_payload(rng, type_id: int, rows: int, cols: int) -> np.ndarray:
    raw = random_payload(rng, type_id, rows, cols)
    name, bs, bpb = TYPES[type_id]
    if type_id in (0, 28, 24, 25, 26, 27):
        return raw
    k = 0
    for blk in range(raw.size // bpb):
        for off in HALF_WORDS.get(type_id, ()):
            h = SPECIAL_HALVES[k % len(SPECIAL_HALVES)]
            raw[blk * bpb + off] = h & 0xFF
            raw[blk * bpb + off + 1] = h >> 8
            k += 1
    return raw


def bits_sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a, dtype="<f8").tobytes()).hexdigest()


def kernel_fixtures(ref) -> None:
    rng = np.random.default_rng(20241201)
    arrays: dict[str, np.ndarray] = {}
    for t, (name, bs, bpb) in TYPES.items():
        cases = {
            "lcg": (2, 512, lcg_payload(t, 2, 512), ref_vector(512)),
            "rand": (3, 512, random_payload(rng, t, 3, 512), rng.standard_normal(512)),
            "special": (3, 512, special_payload(rng, t, 3, 512), rng.standard_normal(512)),
        }
        for case, (rows, cols, payload, x) in cases.items():
            key = f"t{t}_{case}"
            arrays[key + "_payload"] = payload
            arrays[key + "_x"] = x
            arrays[key + "_shape"] = np.array([rows, cols], dtype=np.int64)
            arrays[key + "_matvec"] = ref.matvec(t, payload, x, rows, cols)
            deq = ref.dequantize_rows(t, payload, rows, cols)
            arrays[key + "_dequant_sha"] = np.frombuffer(bytes.fromhex(bits_sha(deq)), dtype=np.uint8)
            if case == "lcg":
                arrays[key + "_dequant"] = deq
    np.savez_compressed(OUT / "native_kernels.npz", **arrays)


def seeded_fixtures(ref) -> None:
    """Config-shaped inputs at reduced row counts (weights N(0,0.02) quantized by
    the oracle encoders; the reference kernel produces the outputs)."""
    o = oracle()
    arrays = {}
    for t, rows, cols, seed in [(12, 8, 1024, 20242001), (14, 8, 1024, 20243001),
                                (2, 4, 1024, 20242101), (7, 4, 1024, 20242102),
                                (8, 4, 1024, 20242103), (11, 4, 1024, 20242104),
                                (13, 4, 1024, 20242105), (23, 4, 1024, 20242106),
                                (14, 4, 768, 20244001), (12, 4, 2048, 20244002)]:
        w = o.normal(seed, rows * cols, 0.0, 0.02).astype(np.float64)
        payload = o.quantize(t, w)
        x = o.normal(seed + 500, cols).astype(np.float64)
        key = f"t{t}_{rows}x{cols}"
        arrays[key + "_payload"] = payload
        arrays[key + "_x"] = x
        arrays[key + "_matvec"] = ref.matvec(t, payload, x, rows, cols)
        arrays[key + "_dequant_sha"] = np.frombuffer(
            bytes.fromhex(bits_sha(ref.dequantize_rows(t, payload, rows, cols))), dtype=np.uint8)
    np.savez_compressed(OUT / "seeded_kernels.npz", **arrays)


def kquant_fixtures() -> None:
    spec = importlib.util.spec_from_file_location("ref_k_quant", REFERENCE_TESTS / "k_quant.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    o = oracle()
    inputs = {
        "sincos": [math.sin(i * 0.071) * 0.6 + math.cos(i * 0.019) * 0.2 for i in range(1024)],
        "normal": [float(v) for v in o.normal(20240101, 1024, 0.0, 0.02)],
        "wide": [float(v) for v in o.normal(20240102, 512, 0.0, 3.0)],
        "pos": [abs(float(v)) + 0.01 for v in o.normal(20240103, 512, 0.0, 0.5)],
    }
    # a block with an all-equal group and one that is entirely zero
    flat = [0.25] * 32 + [float(v) for v in o.normal(20240104, 224, 0.0, 0.1)]
    inputs["flatgroup"] = flat + [0.0] * 256
    arrays = {}
    for name, vals in inputs.items():
        arrays[f"{name}_values"] = np.array(vals, dtype=np.float64)
        for t, enc in mod.K_ENCODERS.items():
            arrays[f"{name}_t{t}"] = np.frombuffer(enc(vals), dtype=np.uint8)
    # pack_q3_k_block on the reference test's own codes/levels (test_ggml_decoders.py:92-108)
    codes = [32 + v for v in (-16, -12, -8, -4, 0, 4, 8, 12, 15, -15, 3, -3, 7, -7, 11, -11)]
    levels = [(i * 3) % 8 for i in range(256)]
    arrays["q3pack_codes"] = np.array(codes, dtype=np.int64)
    arrays["q3pack_levels"] = np.array(levels, dtype=np.int64)
    arrays["q3pack_bytes"] = np.frombuffer(mod.pack_q3_k_block(codes, levels, 0.03125), dtype=np.uint8)
    np.savez_compressed(OUT / "k_quant_vectors.npz", **arrays)


def main() -> None:
    ref = reference()
    if ref is None:
        raise SystemExit("oracle/_ref/libpyrite_ref.so is missing: run `make -C oracle ref` first")
    kernel_fixtures(ref)
    seeded_fixtures(ref)
    kquant_fixtures()
    for p in sorted(OUT.glob("*.npz")):
        print(p.name, p.stat().st_size)


if __name__ == "__main__":
    main()
