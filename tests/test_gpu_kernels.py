"""GPU parity of the dequant and dequant-matvec kernels against the oracle.

Everything goes through the C ABI (include/pyrite_hip.h): the drop-in
pyrite_matvec / pyrite_dequantize_rows via pyrite_amd.native, and the
device-resident pyrite_dev_* entry points via pyrite_amd.device.

Bars: dequantization is bit-exact (fp64 output == reference double; fp32 output
== (float) of it); matvec is within 1e-4 * ||x||_2 * max|row| per row of the
reference's fp64 result.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle.oracle import TYPES, oracle, row_bytes
from tests.gpu_util import announce, assert_matvec_close, f32_bits_equal, f64_bits_equal

pytestmark = pytest.mark.gpu

ALL_TYPES = sorted(TYPES)
CASES = ["lcg", "rand", "special"]


@pytest.fixture(scope="module")
def torch_dev():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    from pyrite_amd import _lib

    _lib.load()  # raises when the HIP library is missing: no silent fallback
    return torch


@pytest.fixture(scope="module")
def golden(golden_dir):
    return np.load(golden_dir / "native_kernels.npz")


def _case(golden, t, case):
    key = f"t{t}_{case}"
    rows, cols = (int(v) for v in golden[key + "_shape"])
    return key, rows, cols, golden[key + "_payload"], golden[key + "_x"]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("t", ALL_TYPES, ids=lambda t: TYPES[t][0])
def test_dropin_dequantize_is_bit_identical(torch_dev, golden, t, case):
    from pyrite_amd import native

    key, rows, cols, payload, _ = _case(golden, t, case)
    announce("dropin_dequant", key, rows, cols)
    got = np.array(native.dequantize_rows(t, payload.tobytes(), rows, cols))
    ref = oracle().dequantize_rows(t, payload, rows, cols)
    assert f64_bits_equal(got, ref)


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("t", ALL_TYPES, ids=lambda t: TYPES[t][0])
def test_device_dequantize_f32_and_f64(torch_dev, golden, t, case):
    torch = torch_dev
    from pyrite_amd import device

    key, rows, cols, payload, _ = _case(golden, t, case)
    announce("device_dequant", key, rows, cols)
    ref = oracle().dequantize_rows(t, payload, rows, cols)
    w = device.upload(payload.tobytes())
    d64 = device.dequantize(t, w, rows, cols, torch.float64).cpu().numpy().ravel()
    d32 = device.dequantize(t, w, rows, cols, torch.float32).cpu().numpy().ravel()
    assert f64_bits_equal(d64, ref)
    assert f32_bits_equal(d32, ref.astype(np.float32))


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("t", ALL_TYPES, ids=lambda t: TYPES[t][0])
def test_dropin_matvec_matches_reference(torch_dev, golden, t, case):
    from pyrite_amd import native

    key, rows, cols, payload, x = _case(golden, t, case)
    announce("dropin_matvec", key, rows, cols)
    got = np.array(native.matvec(t, payload.tobytes(), list(x), rows, cols))
    ref = golden[key + "_matvec"]
    w = oracle().dequantize_rows(t, payload, rows, cols).reshape(rows, cols)
    # fp64 on both sides, different summation order: bounded by n*eps*sum|w*x|
    scale = np.nansum(np.abs(w) * np.abs(x)[None, :], axis=1)
    finite = np.isfinite(ref)
    assert np.all(np.abs(got[finite] - ref[finite]) <= 1e-12 * scale[finite]), key
    assert np.array_equal(np.isnan(got), np.isnan(ref))


def _weights(t, rows, cols, seed):
    o = oracle()
    if TYPES[t][1] == 1:  # plain types: random finite payloads
        rng = np.random.default_rng(seed)
        if t in (0, 28):
            return rng.standard_normal(rows * cols).astype("<f4" if t == 0 else "<f8").view(np.uint8).copy()
        if t == 1:
            return (rng.standard_normal(rows * cols) * 3).astype("<f2").view(np.uint8).copy()
        if t == 30:
            v = rng.standard_normal(rows * cols).astype("<f4").view("<u4") >> 16
            return v.astype("<u2").view(np.uint8).copy()
        return rng.integers(0, 256, rows * row_bytes(t, cols), dtype=np.uint8)
    return o.quantize(t, o.normal(seed, rows * cols, 0.0, 0.02).astype(np.float64))


def _device_matvec_check(torch, t, rows, cols, batch, seed, offset=0):
    from pyrite_amd import device

    o = oracle()
    payload = _weights(t, rows, cols, seed)
    xs = np.stack([o.normal(seed + 1000 + b, cols) for b in range(batch)]).astype(np.float32)
    buf = torch.zeros(payload.size + 16, dtype=torch.uint8, device="cuda")
    buf[offset:offset + payload.size] = torch.from_numpy(payload).cuda()
    w = buf[offset:offset + payload.size]
    y = device.matvec(t, w, torch.from_numpy(xs).cuda(), rows, cols).cpu().numpy()
    wd = o.dequantize_rows(t, payload, rows, cols).reshape(rows, cols)
    rowmax = np.abs(wd).max(axis=1)
    for b in range(batch):
        ref = o.matvec(t, payload, xs[b].astype(np.float64), rows, cols)
        assert_matvec_close(y[b], ref, xs[b], rowmax, f"{TYPES[t][0]} {rows}x{cols} b{b}/{batch} off{offset}")


@pytest.mark.parametrize("batch", [1, 2, 3, 8, 11])
@pytest.mark.parametrize("t", ALL_TYPES, ids=lambda t: TYPES[t][0])
def test_device_matvec_batches(torch_dev, t, batch):
    announce("device_matvec", TYPES[t][0], 37, 1024, batch)
    _device_matvec_check(torch_dev, t, 37, 1024, batch, seed=7000 + t)


@pytest.mark.parametrize("offset", [2, 4, 6])
@pytest.mark.parametrize("t", ALL_TYPES, ids=lambda t: TYPES[t][0])
def test_device_matvec_misaligned_weights(torch_dev, t, offset):
    """Weights that start at any even offset (the verbatim GGUF contract is only
    2-byte alignment per block); plain types need element alignment."""
    from pyrite_amd import _lib

    bpb = TYPES[t][2]
    if TYPES[t][1] == 1 and offset % bpb:
        with pytest.raises(_lib.KernelError) as err:
            _device_matvec_check(torch_dev, t, 5, 256, 1, seed=11, offset=offset)
        assert err.value.code == -3
        return
    announce("device_matvec_misaligned", TYPES[t][0], offset)
    _device_matvec_check(torch_dev, t, 19, 768, 2, seed=8000 + t, offset=offset)


@pytest.mark.parametrize("shape", [(1, 256), (5, 256), (64, 512), (129, 3072), (33, 14336)])
@pytest.mark.parametrize("t", [2, 8, 12, 14, 11, 23, 0], ids=lambda t: TYPES[t][0])
def test_device_matvec_edge_shapes(torch_dev, t, shape):
    rows, cols = shape
    announce("device_matvec_shape", TYPES[t][0], rows, cols)
    _device_matvec_check(torch_dev, t, rows, cols, 1, seed=9000 + rows + t)


# Long rows whose staged activations limit the workgroups per CU: batch-1
# launches run 16-wave workgroups and batch-2 launches 8-wave ones, with more
# than 64 KiB of LDS for the longest; ragged row counts leave partial row
# groups in the last workgroups.
@pytest.mark.parametrize("rows,cols,batch", [(333, 6144, 2), (300, 7936, 2), (1000, 8192, 1), (77, 10240, 1),
                                               (129, 14336, 2), (65, 28672, 1)])
@pytest.mark.parametrize("t", [2, 8, 12, 14, 23], ids=lambda t: TYPES[t][0])
def test_device_matvec_long_rows(torch_dev, t, rows, cols, batch):
    announce("device_matvec_long_rows", TYPES[t][0], rows, cols, batch)
    _device_matvec_check(torch_dev, t, rows, cols, batch, seed=9500 + rows + t)


# The type sweep over the Qwen3-0.6B decode projections at batch 1 and 8.
SWEEP_TYPES = [2, 7, 8, 11, 13, 14, 23]  # Q4_0 Q5_1 Q8_0 Q3_K Q5_K Q6_K IQ4_XS
PROJECTIONS = {"q": (2048, 1024), "k": (1024, 1024), "v": (1024, 1024), "o": (1024, 2048),
               "gate": (3072, 1024), "up": (3072, 1024), "down": (1024, 3072)}


@pytest.mark.parametrize("batch", [1, 8])
@pytest.mark.parametrize("t", SWEEP_TYPES, ids=lambda t: TYPES[t][0])
def test_qwen3_projection_sweep(torch_dev, t, batch):
    for i, (name, (rows, cols)) in enumerate(PROJECTIONS.items()):
        announce("sweep", TYPES[t][0], name, rows, cols, batch)
        _device_matvec_check(torch_dev, t, rows, cols, batch, seed=20242000 + 100 * t + i)


def test_q4_k_config_one(torch_dev):
    """Q4_K 3072 x 1024 from N(0, 0.02), x N(0, 1), batch 1."""
    announce("q4_k 3072x1024 (Qwen3-0.6B ffn_up)")
    _device_matvec_check(torch_dev, 12, 3072, 1024, 1, seed=20241001)


@pytest.mark.parametrize("t,rows,cols", [(12, 14336, 4096), (14, 4096, 14336), (12, 4096, 4096)])
def test_llama_layer_shapes(torch_dev, t, rows, cols):
    announce("llama", TYPES[t][0], rows, cols)
    _device_matvec_check(torch_dev, t, rows, cols, 1, seed=20245000 + rows)


@pytest.mark.parametrize("batch", [1, 8, 64])
@pytest.mark.parametrize("t", [2, 12, 14, 23, 0], ids=lambda t: TYPES[t][0])
def test_grouped_matvec_equals_single_launches(torch_dev, t, batch):
    """pyrite_dev_matvec_grouped over mixed shapes gives, bit for bit, what one
    pyrite_dev_matvec per matrix gives, and both meet the oracle bar."""
    import ctypes

    torch = torch_dev
    from pyrite_amd import _lib, device

    o = oracle()
    lib = _lib.load()
    shapes = [(2048, 1024), (1024, 1024), (1024, 2048), (333, 3072), (7, 256)]
    mats = []
    for i, (rows, cols) in enumerate(shapes):
        payload = _weights(t, rows, cols, 31000 + i)
        x = np.stack([o.normal(32000 + 10 * i + b, cols) for b in range(batch)]).astype(np.float32)
        mats.append((rows, cols, payload, torch.from_numpy(payload).cuda(), torch.from_numpy(x).cuda(), x))
    announce("grouped", TYPES[t][0], batch, len(shapes))

    class Desc(ctypes.Structure):
        _fields_ = [("w", ctypes.c_void_p), ("w_len", ctypes.c_size_t), ("rows", ctypes.c_size_t),
                    ("cols", ctypes.c_size_t), ("x", ctypes.c_void_p), ("ldx", ctypes.c_size_t),
                    ("y", ctypes.c_void_p), ("ldy", ctypes.c_size_t)]

    ys = [torch.full((batch, rows), float("nan"), device="cuda") for rows, *_ in mats]
    arr = (Desc * len(mats))()
    for i, (rows, cols, payload, w, xg, _) in enumerate(mats):
        arr[i] = Desc(w.data_ptr(), payload.nbytes, rows, cols, xg.data_ptr(), cols, ys[i].data_ptr(), rows)
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.pyrite_dev_matvec_grouped(t, arr, len(mats), batch, ctypes.c_void_p(stream)), "grouped")
    for i, (rows, cols, payload, w, xg, x) in enumerate(mats):
        single = device.matvec(t, w, xg, rows, cols)
        assert torch.equal(single, ys[i]), f"matrix {i}"
        rowmax = np.abs(o.dequantize_rows(t, payload, rows, cols).reshape(rows, cols)).max(axis=1)
        got = ys[i].cpu().numpy()
        for b in range(batch):
            ref = o.matvec(t, payload, x[b].astype(np.float64), rows, cols)
            assert_matvec_close(got[b], ref, x[b], rowmax, f"grouped {i} b{b}")


QUANT_TYPES = [t for t in ALL_TYPES if TYPES[t][1] > 1]


def _random_payload(t, rows, cols, seed):
    """Random block bytes (every code, scale and bit pattern) with the fp16
    block scale words kept finite, as in the reference's own kernel test."""
    from tests.gpu_util import random_payload

    return random_payload(np.random.default_rng(seed), t, rows, cols)


@pytest.mark.parametrize("batch", [1, 5, 8])
@pytest.mark.parametrize("t", QUANT_TYPES, ids=lambda t: TYPES[t][0])
def test_device_matvec_random_payloads(torch_dev, t, batch):
    torch = torch_dev
    from pyrite_amd import device

    o = oracle()
    rows, cols = 70, 1024
    payload = _random_payload(t, rows, cols, 4400 + t)
    announce("device_matvec_random", TYPES[t][0], rows, cols, batch)
    xs = np.stack([o.normal(4500 + b, cols) for b in range(batch)]).astype(np.float32)
    y = device.matvec(t, device.upload(payload.tobytes()), torch.from_numpy(xs).cuda(), rows, cols).cpu().numpy()
    wd = o.dequantize_rows(t, payload, rows, cols).reshape(rows, cols)
    rowmax = np.abs(wd).max(axis=1)
    for b in range(batch):
        ref = o.matvec(t, payload, xs[b].astype(np.float64), rows, cols)
        assert_matvec_close(y[b], ref, xs[b], rowmax, f"{TYPES[t][0]} random b{b}/{batch}")


@pytest.mark.parametrize("cols,batch", [(1024, 1), (1024, 8), (4096, 8), (1024, 64), (4096, 70)])
@pytest.mark.parametrize("t", [12, 14, 2, 8], ids=lambda t: TYPES[t][0])
def test_device_matvec_large_activations(torch_dev, t, cols, batch):
    """Activations beyond the fp16 range (|x| up to 3e6) are rescaled by a
    power of two per vector; with 4096 columns at batch 8 the activations are
    staged in several LDS chunks, and batches of 64 and more take the GEMM."""
    torch = torch_dev
    from pyrite_amd import device

    o = oracle()
    rows = 40
    payload = _weights(t, rows, cols, 4600 + cols)
    rng = np.random.default_rng(cols + batch)
    xs = (rng.standard_normal((batch, cols)) * np.where(rng.random((batch, cols)) < 0.01, 1e6, 1.0)).astype(np.float32)
    xs[0, 3] = 3.0e6
    announce("device_matvec_large_x", TYPES[t][0], rows, cols, batch)
    y = device.matvec(t, device.upload(payload.tobytes()), torch.from_numpy(xs).cuda(), rows, cols).cpu().numpy()
    wd = o.dequantize_rows(t, payload, rows, cols).reshape(rows, cols)
    rowmax = np.abs(wd).max(axis=1)
    for b in range(batch):
        ref = o.matvec(t, payload, xs[b].astype(np.float64), rows, cols)
        assert_matvec_close(y[b], ref, xs[b], rowmax, f"{TYPES[t][0]} large-x b{b}/{batch}")


@pytest.mark.parametrize("batch", [1, 8, 64])
@pytest.mark.parametrize("t", [12, 14, 2, 8, 23], ids=lambda t: TYPES[t][0])
def test_device_matvec_activation_scales(torch_dev, t, batch):
    """Each vector scaled by its own power of ten from 1e-30 to 1e30: the fp16
    activation fragments are normalised per vector, so the error stays
    relative to ||x|| at every scale."""
    torch = torch_dev
    from pyrite_amd import device

    o = oracle()
    rows, cols = 48, 2048
    payload = _weights(t, rows, cols, 4700 + t)
    rng = np.random.default_rng(4800 + batch)
    scales = 10.0 ** rng.integers(-30, 31, batch)
    scales[0] = 1e-7
    xs = (np.stack([o.normal(4900 + b, cols) for b in range(batch)]) * scales[:, None]).astype(np.float32)
    announce("device_matvec_scales", TYPES[t][0], rows, cols, batch)
    y = device.matvec(t, device.upload(payload.tobytes()), torch.from_numpy(xs).cuda(), rows, cols).cpu().numpy()
    wd = o.dequantize_rows(t, payload, rows, cols).reshape(rows, cols)
    rowmax = np.abs(wd).max(axis=1)
    for b in range(batch):
        ref = o.matvec(t, payload, xs[b].astype(np.float64), rows, cols)
        assert_matvec_close(y[b], ref, xs[b], rowmax, f"{TYPES[t][0]} scale {scales[b]:g} b{b}/{batch}")


@pytest.mark.parametrize("batch", [64, 100, 130])
@pytest.mark.parametrize("t", QUANT_TYPES, ids=lambda t: TYPES[t][0])
def test_device_matvec_gemm_batches(torch_dev, t, batch):
    """Batches of 64-130 vectors of a 150-row matrix: the dispatcher's cost
    estimate sends 64 vectors of the super-block formats other than Q4_K to
    the chunked MFMA matvec (eight 8-token chunks against weights read once)
    and the rest to the MFMA dequant-GEMM; ragged row and token tiles, every
    vector checked."""
    announce("device_matvec_gemm", TYPES[t][0], 150, 1024, batch)
    _device_matvec_check(torch_dev, t, 150, 1024, batch, seed=9500 + t)


@pytest.mark.parametrize("t,rows,cols,batch", [(12, 4096, 4096, 96), (14, 4096, 4096, 64), (8, 1024, 14336, 72),
                                               (12, 14336, 4096, 33), (12, 14336, 4096, 64), (14, 4096, 4096, 128)])
def test_device_matvec_gemm_llama_shapes(torch_dev, t, rows, cols, batch):
    """Llama-3-8B projection shapes at batches from 33 to 128, on whichever of
    the chunked MFMA matvec and the dequant-GEMM the dispatcher estimates
    faster (Q6_K 4096x4096 at 64 and Q8_0 1024x14336 at 72 take the matvec,
    the others the GEMM)."""
    announce("device_matvec_gemm_llama", TYPES[t][0], rows, cols, batch)
    _device_matvec_check(torch_dev, t, rows, cols, batch, seed=9600 + rows + t)


@pytest.mark.parametrize("batch", [40, 112])
@pytest.mark.parametrize("t", [12, 14], ids=lambda t: TYPES[t][0])
def test_device_matvec_random_payloads_gemm(torch_dev, t, batch):
    """Random block bytes at 40 vectors (chunked MFMA matvec) and 112 (GEMM)."""
    torch = torch_dev
    from pyrite_amd import device

    o = oracle()
    rows, cols = 70, 1024
    payload = _random_payload(t, rows, cols, 4400 + t)
    announce("device_matvec_random_gemm", TYPES[t][0], rows, cols, batch)
    xs = np.stack([o.normal(4500 + b, cols) for b in range(batch)]).astype(np.float32)
    y = device.matvec(t, device.upload(payload.tobytes()), torch.from_numpy(xs).cuda(), rows, cols).cpu().numpy()
    wd = o.dequantize_rows(t, payload, rows, cols).reshape(rows, cols)
    rowmax = np.abs(wd).max(axis=1)
    for b in range(batch):
        ref = o.matvec(t, payload, xs[b].astype(np.float64), rows, cols)
        assert_matvec_close(y[b], ref, xs[b], rowmax, f"{TYPES[t][0]} random b{b}/{batch}")


@pytest.mark.parametrize("batch", [1, 2, 5])
@pytest.mark.parametrize("t", [12, 14, 2, 8, 23, 0], ids=lambda t: TYPES[t][0])
def test_device_matvec_nonfinite_activations(torch_dev, t, batch):
    """An infinite or NaN activation in one vector: the rows it reaches are
    non-finite, as in the reference (which of inf and NaN may differ: the
    kernels factor the block scales out of the sums, so 0 * inf can appear
    where the reference multiplies a dequantized weight), and every finite
    reference row is within the bar."""
    torch = torch_dev
    from pyrite_amd import device

    o = oracle()
    rows, cols = 40, 512
    payload = _weights(t, rows, cols, 4950 + t)
    xs = np.stack([o.normal(4960 + b, cols) for b in range(batch)]).astype(np.float32)
    xs[0, 7] = np.float32(np.inf)
    if batch > 1:
        xs[1, 100] = np.float32(np.nan)
    announce("device_matvec_nonfinite", TYPES[t][0], rows, cols, batch)
    y = device.matvec(t, device.upload(payload.tobytes()), torch.from_numpy(xs).cuda(), rows, cols).cpu().numpy()
    wd = o.dequantize_rows(t, payload, rows, cols).reshape(rows, cols)
    rowmax = np.abs(wd).max(axis=1)
    for b in range(batch):
        ref = o.matvec(t, payload, xs[b].astype(np.float64), rows, cols)
        assert np.array_equal(np.isfinite(y[b]), np.isfinite(ref)), f"b{b}: finite rows differ"
        fin = np.isfinite(ref)
        if fin.any():
            err = np.abs(y[b][fin].astype(np.float64) - ref[fin])
            xf = np.where(np.isfinite(xs[b]), xs[b], 0.0)
            assert np.all(err <= 1e-4 * np.linalg.norm(xf) * rowmax[fin]), f"b{b}: finite rows off"


# The 512-token prefill of one Llama-3-8B layer in the Q4_K_M mix (the MFMA
# dequant-GEMM: 16 token tiles of 32).  Tokens checked against the oracle:
# every token of the first and the last token tile and every 8th token between.
LLAMA_LAYER = [("q", 12, 4096, 4096), ("k", 12, 1024, 4096), ("v", 12, 1024, 4096), ("o", 12, 4096, 4096),
               ("gate", 12, 14336, 4096), ("up", 12, 14336, 4096), ("down", 14, 4096, 14336)]
PREFILL_TOKENS = sorted(set(range(32)) | set(range(480, 512)) | set(range(0, 512, 8)))
_PREFILL_PAYLOADS: dict = {}


@pytest.mark.parametrize("name,t,rows,cols", LLAMA_LAYER, ids=[m[0] for m in LLAMA_LAYER])
def test_llama_layer_prefill_512(torch_dev, name, t, rows, cols):
    from concurrent.futures import ThreadPoolExecutor

    from pyrite_amd import device

    torch = torch_dev
    o = oracle()
    seed = 20245500 + rows + cols
    if (t, rows, cols) not in _PREFILL_PAYLOADS:  # q/o, k/v and gate/up share their weights
        _PREFILL_PAYLOADS[(t, rows, cols)] = o.quantize(t, o.normal(seed, rows * cols, 0.0, 0.02).astype(np.float64))
    payload = _PREFILL_PAYLOADS[(t, rows, cols)]
    xs = np.stack([o.normal(seed + 1 + b, cols) for b in range(512)]).astype(np.float32)
    announce("llama_prefill_512", name, TYPES[t][0], rows, cols, 512)
    y = device.matvec(t, device.upload(payload.tobytes()), torch.from_numpy(xs).cuda(), rows, cols).cpu().numpy()
    rb = row_bytes(t, cols)
    rowmax = np.concatenate([
        np.abs(o.dequantize_rows(t, payload[r0 * rb:min(rows, r0 + 1024) * rb], min(1024, rows - r0), cols)
               .reshape(-1, cols)).max(axis=1) for r0 in range(0, rows, 1024)])

    def ref(b):  # the oracle call releases the GIL
        return b, o.matvec(t, payload, xs[b].astype(np.float64), rows, cols)

    with ThreadPoolExecutor(8) as pool:
        for b, r in pool.map(ref, PREFILL_TOKENS):
            assert_matvec_close(y[b], r, xs[b], rowmax, f"prefill {name} {rows}x{cols} token {b}/512")
