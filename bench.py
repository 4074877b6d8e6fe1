#!/usr/bin/env python3
"""Benchmark of the fused GGML dequantize x matvec path on one MI355X.

Headline workload (value, roofline): the batch-1 decode of one Llama-3-8B
layer in the Q4_K_M mix -- attn q/o 4096x4096 and k/v 1024x4096, ffn gate/up
14336x4096 in Q4_K, ffn down 4096x14336 in Q6_K (137.8 MB of quantized
weights), each quantized from seeded N(0, 0.02) fp32 weights, with fp32
N(0, 1) activations.  One step is the layer's four launches in executor
order: q/k/v grouped (pyrite_dev_matvec_grouped), o, gate/up grouped, down.
Weights are uploaded verbatim and rotated over 3 device copies (413 MB > the
256 MB Infinity Cache), so every launch reads its weights from HBM.  The
timed steps are captured into one HIP graph and replayed once between two
synchronisations.  value = quantized weight bytes / second over the timed
steps (GB/s).  Each launch's duration for the roofline comes from HIP events
that the launch itself records at kernel start and end (hipExtLaunchKernelGGL),
over the same launches replayed eagerly on the same stream.

Under "workloads", every other configuration of the path, each with its own
roofline object: the single Q4_K 3072x1024 matvec, the Qwen3-0.6B projection
type sweep (7 types x 7 projections, batch 1 and 8), the Q6_K 151936x1024 LM
head with its exact greedy id, the Qwen3-30B-A3B MoE layer (tokens/s at batch
1, 8, 64; also at top level), the Llama-3-8B layer's matrices alone at batch 1
and its 512-token prefill (MFMA dequant-GEMM, against the fp16 matrix-core
peak), and the GGUF -> HBM upload rate of the resident-tensor loader.

cpu_baseline: the reference's own native.c (oracle/_ref, built from the
reference source) timed on the host on a bounded sample of the headline
workload (whole decode layers, 7 single-vector pyrite_matvec calls each) by
the C harness oracle/cpu_bench.c: one warm-up pass, median of 5 timed runs,
on one thread and on all host cores (at most 16).

Prints one JSON line.  --gpus N > 1 exits: this path runs on one GPU.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense fp16 matrix-core peak (the dequant-GEMM runs f16 MFMAs)
LLAMA = [("q", 12, 4096, 4096), ("k", 12, 1024, 4096), ("v", 12, 1024, 4096), ("o", 12, 4096, 4096),
         ("gate", 12, 14336, 4096), ("up", 12, 14336, 4096), ("down", 14, 4096, 14336)]
# the decode step's launches: (name, type, matrices, activation)
DECODE_LAUNCHES = [("qkv", 12, ("q", "k", "v"), "normed"), ("o", 12, ("o",), "attn"),
                   ("gate_up", 12, ("gate", "up"), "normed2"), ("down", 14, ("down",), "act")]
DECODE_COPIES = 3
SWEEP_TYPES = [("Q4_0", 2), ("Q5_1", 7), ("Q8_0", 8), ("Q3_K", 11), ("Q5_K", 13), ("Q6_K", 14), ("IQ4_XS", 23)]
PROJECTIONS = [("q", 2048, 1024), ("k", 1024, 1024), ("v", 1024, 1024), ("o", 1024, 2048),
               ("gate", 3072, 1024), ("up", 3072, 1024), ("down", 1024, 3072)]
BATCHES = (1, 8)
COPIES = 4
SEED = 20241201


class Desc(ctypes.Structure):
    """pyrite_matvec_desc (include/pyrite_hip.h)."""

    _fields_ = [("w", ctypes.c_void_p), ("w_len", ctypes.c_size_t), ("rows", ctypes.c_size_t),
                ("cols", ctypes.c_size_t), ("x", ctypes.c_void_p), ("ldx", ctypes.c_size_t),
                ("y", ctypes.c_void_p), ("ldy", ctypes.c_size_t)]


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_info() -> tuple[str, int]:
    model = platform.processor() or "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return model, os.cpu_count() or 1


def roofline_hbm(nbytes: float, avg_s: float, traffic=None, **extra) -> dict:
    """Roofline object of an HBM-bound launch: algorithmic bytes per launch / its average duration."""
    gbs = nbytes / avg_s / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic, "bytes_per_launch": int(nbytes),
            "avg_launch_us": round(avg_s * 1e6, 3), **extra}


def load_traffic(profile: str, key: str):
    """HBM bytes per launch of `key` from a committed FETCH_SIZE / WRITE_SIZE
    summary (profiles/<profile>.json), or None."""
    try:
        data = json.loads((ROOT / "profiles" / f"{profile}.json").read_text())
    except (OSError, ValueError):
        return None
    entry = data.get("launches", {}).get(key)
    return None if entry is None else entry.get("hbm_bytes_per_launch")


def llama_weights(np, quantize):
    """The Llama-3-8B layer's matrices {name: (type, rows, cols, payload)}; matrices of
    one shape and type share their seeded weights (q/o, k/v, gate/up)."""
    cache, out = {}, {}
    for name, t, rows, cols in LLAMA:
        key = (t, rows, cols)
        if key not in cache:
            cache[key] = quantized_normal(np, quantize, t, rows * cols, SEED + 20 + len(cache))
        out[name] = (t, rows, cols, cache[key])
    return out


def run_cpu_baseline(np, calls, budget_s: float, nthreads: int, what: str, runs: int = 5):
    """Time the reference's scalar fp64 pyrite_matvec (oracle/_ref; the oracle's
    restatement when that build is absent) over `calls` [(type, payload, x, rows,
    cols)] with the C harness oracle/cpu_bench.c: one warm-up pass, then `runs`
    timed runs of P passes each (P sized so the runs take about budget_s), the
    median run reported; no Python in the timed region.  With nthreads > 1,
    thread i runs every call on its own i-th share of each matrix's rows."""
    import ctypes

    from oracle.oracle import oracle, reference

    impl = reference()
    kind = "reference"
    if impl is None:
        impl = oracle()
        kind = "port"
    h = ctypes.CDLL(str(ROOT / "oracle" / "libcpubench.so"))
    sz, vp = ctypes.c_size_t, ctypes.c_void_p
    h.cpu_bench_run.restype = ctypes.c_int
    h.cpu_bench_run.argtypes = [vp, ctypes.c_int, vp, vp, vp, vp, vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                vp]
    n = len(calls)
    payloads = [np.ascontiguousarray(p, dtype=np.uint8) for _, p, _, _, _ in calls]
    xs = [np.ascontiguousarray(x, dtype=np.float64) for _, _, x, _, _ in calls]
    types = np.array([t for t, *_ in calls], dtype=np.int32)
    rows = np.array([r for *_, r, _ in calls], dtype=np.uint64)
    cols = np.array([c for *_, c in calls], dtype=np.uint64)
    rbytes = np.array([p.nbytes // r for p, r in zip(payloads, rows)], dtype=np.uint64)
    wptr = np.array([p.ctypes.data for p in payloads], dtype=np.uint64)
    xptr = np.array([x.ctypes.data for x in xs], dtype=np.uint64)
    fn = ctypes.cast(impl._mv, vp).value

    def timed(nruns, passes):
        out = np.zeros(nruns, dtype=np.float64)
        rc = h.cpu_bench_run(fn, n, types.ctypes.data, wptr.ctypes.data, rows.ctypes.data, cols.ctypes.data,
                             rbytes.ctypes.data, xptr.ctypes.data, nthreads, nruns, passes, out.ctypes.data)
        if rc != 0:
            raise RuntimeError(f"cpu_bench_run failed: {rc}")
        return out

    one = float(timed(1, 1)[0])  # calibration: one pass
    passes = max(1, int(round(budget_s / runs / max(one, 1e-6))))
    run_s = timed(runs, passes)
    med = float(np.median(run_s))
    bytes_per_pass = sum(p.nbytes for p in payloads)
    return {"value": bytes_per_pass * passes / med / 1e9, "unit": "GB/s", "cores": nthreads, "kind": kind,
            "sample": f"median of {runs} timed runs of {passes} pass(es) of {what} through pyrite_matvec "
                      f"(runs {run_s.min():.2f}-{run_s.max():.2f} s, one warm-up pass), "
                      + ("single thread" if nthreads == 1 else
                         f"{nthreads} threads, thread i on its i-th share of every matrix's rows")
                      + ", C harness oracle/cpu_bench.c"}


def timed_grouped(lib, stream, sptr, launches, steps):
    """Average kernel seconds of each grouped launch: launches = [(key, type, desc arrays per step
    (callable s -> (array, n)), batch)], run eagerly for `steps` steps, each timed by HIP events
    that the launch itself records at kernel start and end (pyrite_dev_matvec_grouped_timed)."""
    import torch

    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in launches]
    for pair in evs:
        for e in pair:
            e.record(stream)  # creates the underlying hipEvent_t
    torch.cuda.synchronize()
    durations = {key: [] for key, *_ in launches}
    for s in range(steps):
        for k, (key, t, descs, batch) in enumerate(launches):
            arr, n = descs(s)
            rc = lib.pyrite_dev_matvec_grouped_timed(t, arr, n, batch, sptr, ctypes.c_void_p(evs[k][0].cuda_event),
                                                     ctypes.c_void_p(evs[k][1].cuda_event))
            if rc != 0:
                raise RuntimeError(f"timed launch {key} failed: {rc} {lib.pyrite_hip_last_error()}")
        torch.cuda.synchronize()
        for k, (key, *_) in enumerate(launches):
            durations[key].append(evs[k][0].elapsed_time(evs[k][1]) * 1e-3)
    return {key: sum(d) / len(d) for key, d in durations.items()}


TIMING = ("HIP events recorded by each launch at kernel start/end (hipExtLaunchKernelGGL), same launches "
          "and weight rotation as the timed graph, on the same stream")


# ---------------------------------------------------------------- other configurations
# Each is timed as `reps` calls captured in one HIP graph (replayed once after
# a warm-up replay), over rotated weight copies or varying inputs so that
# weights come from HBM rather than the 256 MB Infinity Cache.

def time_graph(torch, stream, calls, check=None) -> float:
    """Seconds per call for a list of zero-argument callables captured in one graph."""
    for c in (calls if check else calls[:2]):
        c()  # eager warm-up (workspaces are sized outside capture) and the reference for the check
    torch.cuda.synchronize()
    eager = check() if check else None
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for c in calls:
            c()
    g.replay()
    torch.cuda.synchronize()
    if check is not None:
        again = check()
        for a, b in zip(eager, again):
            if not torch.equal(a, b):
                raise RuntimeError("graph replay differs from the eager calls")
    t0 = time.perf_counter()
    g.replay()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / len(calls)


def quantized_normal(np, quantize, t, n, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal(n, dtype=np.float32) * np.float32(0.02)).astype(np.float64)
    return quantize(t, w)


COPY_BYTES = 256 << 20


def copy_calibration(torch, stream):
    """Plain device copies of 256 MiB (read 256 MiB, write 256 MiB per copy):
    the known-size reference for scaling the FETCH_SIZE / WRITE_SIZE counters."""
    src = torch.randn(COPY_BYTES // 4, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    return {"workload": "torch copy_ of 256 MiB fp32, 5 times", "read_bytes_per_copy": COPY_BYTES,
            "write_bytes_per_copy": COPY_BYTES}


def launch_kernel_name(batch: int) -> str:
    """Kernel that a grouped launch of a block format runs at this batch."""
    return "mg_kernel (MFMA dequant-GEMM)" if batch >= 64 else "mx_kernel (MFMA)" if batch >= 3 else \
        "mv_kernel (VALU)"


def bench_gguf_upload(torch, np):
    """GGUF file -> HBM: pyrite_amd.resident.ResidentTensors over a 4-layer
    Llama-3-8B Q4_K_M-shaped checkpoint (551 MB of tensor bytes) written to a
    temporary file just before, so the file is read from the page cache."""
    import shutil
    import struct
    import tempfile

    from pyrite_amd.gguf import GGUFReader
    from pyrite_amd.resident import ResidentTensors

    shapes = [("attn_q", 12, 4096, 4096), ("attn_k", 12, 1024, 4096), ("attn_v", 12, 1024, 4096),
              ("attn_output", 12, 4096, 4096), ("ffn_gate", 12, 14336, 4096), ("ffn_up", 12, 14336, 4096),
              ("ffn_down", 14, 4096, 14336)]
    bpb = {12: (256, 144), 14: (256, 210)}
    tensors = []
    for layer in range(4):
        for name, t, rows, cols in shapes:
            bs, b = bpb[t]
            tensors.append((f"blk.{layer}.{name}.weight", (cols, rows), t, rows * (cols // bs) * b))

    def s(text):
        raw = text.encode()
        return struct.pack("<Q", len(raw)) + raw

    align = 32
    meta = s("general.alignment") + struct.pack("<II", 4, align)
    offs, off = [], 0
    for _, _, _, n in tensors:
        offs.append(off)
        off = -(-(off + n) // align) * align
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), 1) + meta
    for (name, dims, t, _), o in zip(tensors, offs):
        head += s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", t, o)
    head += bytes(-len(head) % align)
    rng = np.random.default_rng(SEED + 40)
    chunk = rng.integers(0, 256, size=1 << 24, dtype=np.uint8)  # 16 MiB pattern, rotated per tensor
    tmp = Path(tempfile.mkdtemp(prefix="pyrite_gguf_"))
    path = tmp / "llama3_8b_4layers.gguf"
    try:
        with path.open("wb") as fh:
            fh.write(head)
            pos = 0
            for i, ((_, _, _, n), o) in enumerate(zip(tensors, offs)):
                fh.write(bytes(o - pos))
                pattern = np.roll(chunk, 4099 * i)  # a different byte pattern per tensor
                k = 0
                while k < n:
                    m = min(n - k, pattern.size)
                    fh.write(pattern[:m].tobytes())
                    k += m
                pos = o + n
        total = sum(n for *_, n in tensors)
        times = []
        for _ in range(2):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            res = ResidentTensors(GGUFReader(path))
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t0)
        # the uploaded bytes are the file's (first MiB of every tensor)
        reader = GGUFReader(path)
        for tinfo in reader.tensor_index():
            with path.open("rb") as fh:
                fh.seek(tinfo.offset)
                want = np.frombuffer(fh.read(1 << 20), dtype=np.uint8)
            if not np.array_equal(res.view(tinfo.name)[:want.size].cpu().numpy(), want):
                raise RuntimeError(f"uploaded bytes of {tinfo.name} differ from the file")
        del res
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    best = min(times)
    return {"workload": "GGUF -> HBM upload (ResidentTensors), 4 Llama-3-8B Q4_K_M layers, page-cached file",
            "bytes": total, "seconds": round(best, 4), "gbs": round(total / best / 1e9, 2),
            "first_call_seconds": round(times[0], 4)}


def _descs(np, mats, x, ys, copies=None):
    """A Desc array over mats [(t, rows, cols, payload)] with device weights `copies`
    (or their first copy), input x [batch, cols] and outputs ys."""
    arr = (Desc * len(mats))()
    for i, ((t, rows, cols, payload), w, y) in enumerate(zip(mats, copies, ys)):
        arr[i] = Desc(w.data_ptr(), payload.nbytes, rows, cols, x.data_ptr(), x.stride(0) if x.shape[0] > 1 else cols,
                      y.data_ptr(), y.stride(0) if y.shape[0] > 1 else rows)
    return arr


def bench_q4k_single(torch, np, quantize, lib, stream, sptr, device):
    """Single Q4_K 3072x1024 matvec (Qwen3-0.6B ffn_up), batch 1."""
    rows, cols = 3072, 1024
    p = quantized_normal(np, quantize, 12, rows * cols, SEED + 11)
    ws = [torch.from_numpy(p).cuda() for _ in range(160)]  # 283 MB of copies
    x = torch.randn(1, cols, device="cuda")
    y = torch.empty(1, rows, device="cuda")
    calls = [lambda w=w: device.matvec(12, w, x, rows, cols, out=y) for w in ws]
    dt = time_graph(torch, stream, calls)
    arrs = [_descs(np, [(12, rows, cols, p)], x, [y], [w]) for w in ws]
    avg = timed_grouped(lib, stream, sptr, [("q4k", 12, lambda s: (arrs[s % len(arrs)], 1), 1)], len(arrs))["q4k"]
    return {"workload": "Q4_K 3072x1024 matvec, batch 1", "us": round(dt * 1e6, 3),
            "gbs": round(p.nbytes / dt / 1e9, 1), "pct_hbm_peak": round(100 * p.nbytes / dt / 1e9 / HBM_PEAK_GBS, 2),
            "roofline": roofline_hbm(p.nbytes, avg, load_traffic("traffic_configs", "q4k_3072x1024"),
                                     kernel="mv_kernel (VALU) Q4_K batch 1", timing=TIMING)}


def bench_sweep(torch, np, quantize, lib, stream, sptr, steps: int):
    """Qwen3-0.6B projection type sweep: one grouped launch of the 7 projections per type and batch."""
    rng = np.random.default_rng(SEED)
    weights = {}
    for _, t in SWEEP_TYPES:
        mats = []
        for _, rows, cols in PROJECTIONS:
            w = (rng.standard_normal(rows * cols, dtype=np.float32) * np.float32(0.02)).astype(np.float64)
            payload = quantize(t, w)
            base = torch.from_numpy(payload).cuda()
            mats.append(((t, rows, cols, payload), [base] + [base.clone() for _ in range(COPIES - 1)]))
        weights[t] = mats
    xs = {(cols, b): torch.randn(b, cols, device="cuda") for cols in {c for _, _, c in PROJECTIONS} for b in BATCHES}
    ys = {(t, i, b): torch.empty(b, rows, device="cuda")
          for _, t in SWEEP_TYPES for i, (_, rows, _c) in enumerate(PROJECTIONS) for b in BATCHES}
    descs = {}
    for _, t in SWEEP_TYPES:
        for b in BATCHES:
            for c in range(COPIES):
                arr = (Desc * len(PROJECTIONS))()
                for i, ((tt, rows, cols, payload), copies) in enumerate(weights[t]):
                    x, y = xs[(cols, b)], ys[(t, i, b)]
                    arr[i] = Desc(copies[c].data_ptr(), payload.nbytes, rows, cols, x.data_ptr(), cols,
                                  y.data_ptr(), rows)
                descs[(t, b, c)] = arr
    launches = [(t, b) for b in BATCHES for _, t in SWEEP_TYPES]

    def step(s):
        for t, b in launches:
            rc = lib.pyrite_dev_matvec_grouped(t, descs[(t, b, (2 * s + BATCHES.index(b)) % COPIES)],
                                               len(PROJECTIONS), b, sptr)
            if rc != 0:
                raise RuntimeError(f"sweep launch ({t}, {b}) failed: {rc} {lib.pyrite_hip_last_error()}")
    dt = time_graph(torch, stream, [lambda s=s: step(s) for s in range(steps)],
                    check=lambda: [y.clone() for y in ys.values()])
    bytes_per_set = sum(m[0][3].nbytes for mats in weights.values() for m in mats)
    names = dict((v, n) for n, v in SWEEP_TYPES)
    avg = timed_grouped(lib, stream, sptr,
                        [(f"{names[t]}_b{b}", t, lambda s, t=t, b=b: (descs[(t, b, (2 * s + BATCHES.index(b)) % COPIES)],
                                                                     len(PROJECTIONS)), b) for t, b in launches],
                        steps)
    per = {}
    for t, b in launches:
        key = f"{names[t]}_b{b}"
        nbytes = sum(m[0][3].nbytes for m in weights[t])
        per[key] = {"avg_us": round(avg[key] * 1e6, 3), "bytes_per_launch": nbytes,
                    "gbs": round(nbytes / avg[key] / 1e9, 1), "pct_hbm_peak": round(100 * nbytes / avg[key] / 8e12, 2)}
    dom = max(per, key=lambda k: per[k]["avg_us"])
    return {"workload": "Qwen3-0.6B decode projection type sweep: q 2048x1024, k/v 1024x1024, o 1024x2048, "
                        "gate/up 3072x1024, down 1024x3072 x {Q4_0,Q5_1,Q8_0,Q3_K,Q5_K,Q6_K,IQ4_XS} x batch {1,8}, "
                        f"one grouped launch per type and batch, {COPIES} weight copies",
            "ms_per_sweep": round(dt * 1e3, 4), "gbs": round(bytes_per_set * len(BATCHES) / dt / 1e9, 1),
            "per_launch": per,
            "roofline": roofline_hbm(per[dom]["bytes_per_launch"], avg[dom], load_traffic("traffic_sweep", dom),
                                     kernel=f"{launch_kernel_name(int(dom.rsplit('_b', 1)[1]))} {dom}", timing=TIMING)}


def bench_lm_head(torch, np, quantize, lib, stream, sptr, device):
    """Qwen3 LM head: Q6_K 151936x1024, RMS-normalised N(0,1) input, logits + greedy id."""
    rows, cols = 151936, 1024
    p = quantized_normal(np, quantize, 14, rows * cols, SEED + 12)
    ws = [torch.from_numpy(p).cuda() for _ in range(3)]
    rng = np.random.default_rng(SEED + 13)
    xs = []
    for _ in range(6):
        h = rng.standard_normal(cols)
        xs.append(torch.from_numpy((h / np.sqrt(np.mean(h * h) + 1e-6)).astype(np.float32)[None, :]).cuda())
    logits = torch.empty(1, rows, device="cuda")
    ids = []

    def head(i):
        _, idt = device.lm_head_argmax(14, ws[i % 3], xs[i % 6], rows, cols, logits=logits)
        ids.append(idt)
    reps = 24
    dt_head = time_graph(torch, stream, [lambda i=i: head(i) for i in range(reps)])
    dt_mv = time_graph(torch, stream, [lambda i=i: device.matvec(14, ws[i % 3], xs[i % 6], rows, cols, out=logits)
                                       for i in range(reps)])
    arrs = [_descs(np, [(14, rows, cols, p)], xs[i % 6], [logits], [ws[i % 3]]) for i in range(6)]
    avg = timed_grouped(lib, stream, sptr, [("head", 14, lambda s: (arrs[s % 6], 1), 1)], 24)["head"]
    return {"workload": "Q6_K 151936x1024 LM head, batch 1 (logits + exact greedy id)",
            "us_per_token": round(dt_head * 1e6, 2), "tokens_per_s": round(1 / dt_head, 1),
            "gbs": round(p.nbytes / dt_head / 1e9, 1),
            "pct_hbm_peak": round(100 * p.nbytes / dt_head / 1e9 / HBM_PEAK_GBS, 2),
            "matvec_only_us": round(dt_mv * 1e6, 2), "matvec_only_gbs": round(p.nbytes / dt_mv / 1e9, 1),
            "bytes_per_token": p.nbytes,
            "roofline": roofline_hbm(p.nbytes, avg, load_traffic("traffic_configs", "lm_head_matvec"),
                                     kernel="mv_kernel (VALU) Q6_K batch 1, the logits matvec", timing=TIMING),
            "roofline_with_id": roofline_hbm(p.nbytes, dt_head, load_traffic("traffic_configs", "lm_head_with_id"),
                                             kernel="lm_fused_kernel per token (bound matvec; its last "
                                                    "workgroup decides the exact id)",
                                             timing="graph replay per token (the launch and the gap to the next)")}


def bench_moe(torch, np, quantize, stream, device, distinct_experts: int = 8):
    """Qwen3-30B-A3B MoE FFN: 128 experts, hidden 2048, inter 768, top-8; batch 1, 8, 64."""
    E, H, I, K = 128, 2048, 768, 8
    rng = np.random.default_rng(SEED + 14)
    router = (rng.standard_normal(E * H, dtype=np.float32) * np.float32(0.02)).view(np.uint8).copy()
    # distinct_experts seeded quantized experts, tiled over the 128 expert slices
    g = [quantized_normal(np, quantize, 12, I * H, SEED + 100 + e) for e in range(distinct_experts)]
    u = [quantized_normal(np, quantize, 12, I * H, SEED + 200 + e) for e in range(distinct_experts)]
    d = [quantized_normal(np, quantize, 14, H * I, SEED + 300 + e) for e in range(distinct_experts)]
    gate = np.concatenate([g[e % distinct_experts] for e in range(E)])
    up = np.concatenate([u[e % distinct_experts] for e in range(E)])
    down = np.concatenate([d[e % distinct_experts] for e in range(E)])
    slice_bytes = g[0].nbytes + u[0].nbytes + d[0].nbytes
    layers = []
    for _ in range(2):  # two copies of the whole layer (862 MB), alternated
        layers.append(device.MoeLayer(0, torch.from_numpy(router).cuda(), 12, torch.from_numpy(gate).cuda(),
                                      12, torch.from_numpy(up).cuda(), 14, torch.from_numpy(down).cuda(),
                                      E, H, I, K, True, 1.0))
    out = {}
    for batch in (1, 8, 64):
        reps = 16
        xs = [torch.from_numpy(rng.standard_normal((batch, H), dtype=np.float32)).cuda() for _ in range(reps)]
        ys = [torch.empty(batch, H, device="cuda") for _ in range(reps)]
        holder = {}

        def call(i):
            _, ids, _ = device.moe_ffn(layers[i % 2], xs[i], out=ys[i])
            holder[i] = ids
        dt = time_graph(torch, stream, [lambda i=i: call(i) for i in range(reps)], check=lambda: [y.clone() for y in ys])
        distinct = [len(set(holder[i].cpu().numpy().reshape(-1).tolist())) for i in range(reps)]
        nbytes = float(np.mean(distinct)) * slice_bytes + router.nbytes
        out[f"b{batch}"] = {"us_per_layer": round(dt * 1e6, 2), "tokens_per_s": round(batch / dt, 1),
                            "distinct_experts": round(float(np.mean(distinct)), 2),
                            "gbs": round(nbytes / dt / 1e9, 1),
                            "pct_hbm_peak": round(100 * nbytes / dt / 1e9 / HBM_PEAK_GBS, 2),
                            "roofline": roofline_hbm(nbytes, dt, load_traffic("traffic_configs", f"moe_b{batch}"),
                                                     kernel="router, routing, gate/up, down and combine launches",
                                                     timing="graph replay per layer call (all launches and the "
                                                            "gaps between them); bytes = router + the distinct "
                                                            "experts' gate/up/down slices")}
    out["workload"] = ("Qwen3-30B-A3B MoE FFN layer: router F32 2048x128, gate/up Q4_K [128x768x2048], "
                       f"down Q6_K [128x2048x768], top-8, renormalised; {distinct_experts} seeded quantized "
                       "experts tiled over the 128 slices, 2 layer copies alternated, distinct inputs per call")
    return out


def llama_step_descs(np, torch, mats, batch, copies):
    """Desc arrays of the layer's four launches for each weight copy, and the inputs/outputs."""
    xs = {"normed": torch.randn(batch, 4096, device="cuda"), "attn": torch.randn(batch, 4096, device="cuda"),
          "normed2": torch.randn(batch, 4096, device="cuda"), "act": torch.randn(batch, 14336, device="cuda")}
    ys = {name: torch.empty(batch, rows, device="cuda") for name, (t, rows, cols, p) in mats.items()}
    arrs = {}
    for key, t, names, xname in DECODE_LAUNCHES:
        for c in range(len(copies)):
            arrs[(key, c)] = _descs(np, [mats[n] for n in names], xs[xname], [ys[n] for n in names],
                                    [copies[c][n] for n in names])
    return arrs, xs, ys


def run_llama_step(lib, sptr, arrs, batch, c):
    for key, t, names, _ in DECODE_LAUNCHES:
        rc = lib.pyrite_dev_matvec_grouped(t, arrs[(key, c)], len(names), batch, sptr)
        if rc != 0:
            raise RuntimeError(f"{key} launch failed: {rc} {lib.pyrite_hip_last_error()}")


LLAMA_WORKLOAD = ("Llama-3-8B layer, Q4_K_M mix: q/o 4096x4096, k/v 1024x4096, gate/up 14336x4096 Q4_K, "
                  "down 4096x14336 Q6_K")


def bench_llama(torch, np, quantize, stream, device, lib, sptr, mats):
    """Llama-3-8B layer in Q4_K_M mix: its q, gate and down matrices alone at batch 1
    and at 8-96 vectors, and the 512-token prefill (four launches, MFMA dequant-GEMM)."""
    res = {"workload": LLAMA_WORKLOAD, "bytes_per_layer": sum(p.nbytes for _, _, _, p in mats.values())}
    res["prefill_512"] = bench_llama_prefill(torch, np, stream, lib, sptr, mats)
    res["decode_b1_matrices"] = bench_llama_singles(torch, np, stream, device, lib, sptr, mats)
    res["multi_vector_matrices"] = bench_llama_batches(torch, np, stream, device, mats)
    return res


def bench_llama_batches(torch, np, stream, device, mats, batches=(8, 16, 32, 48, 63, 96)):
    """The layer's q, gate and down matrices at several vectors per call (batched decode
    of that many sequences), over rotated copies beyond the Infinity Cache: the MFMA
    matvec (each weight read once for all the 8-token chunks) or the dequant-GEMM,
    whichever the library's estimate picks for the matrix and batch."""
    out = {}
    for name in ("q", "gate", "down"):
        t, rows, cols, p = mats[name]
        n = max(2, int(np.ceil(600e6 / p.nbytes)))
        first = torch.from_numpy(p).cuda()
        ws = [first] + [first.clone() for _ in range(n - 1)]
        label = {12: "Q4_K", 14: "Q6_K"}[t]
        per = {}
        for b in batches:
            x = torch.randn(b, cols, device="cuda")
            y = torch.empty(b, rows, device="cuda")
            dt = time_graph(torch, stream, [lambda w=w: device.matvec(t, w, x, rows, cols, out=y) for w in ws * 2])
            per[f"b{b}"] = {"us": round(dt * 1e6, 2), "weight_gbs": round(p.nbytes / dt / 1e9, 1),
                            "vectors_per_s": round(b / dt, 1)}
        out[f"{name} {rows}x{cols} {label}"] = per
        del ws, first
        torch.cuda.empty_cache()
    return out


def bench_llama_prefill(torch, np, stream, lib, sptr, mats):
    """The layer's 512-token prefill: four grouped launches (MFMA dequant-GEMM)."""
    # 2 weight copies, 2 steps per graph
    copies = [{n: torch.from_numpy(m[3]).cuda() for n, m in mats.items()} for _ in range(2)]
    batch = 512
    arrs, xs, ys = llama_step_descs(np, torch, mats, batch, copies)
    dt = time_graph(torch, stream, [lambda c=c: run_llama_step(lib, sptr, arrs, batch, c) for c in (0, 1)])
    flops = 2.0 * batch * sum(r * c for _, r, c, _ in mats.values())
    avg = timed_grouped(lib, stream, sptr, [(key, t, lambda s, key=key, names=names: (arrs[(key, s % 2)], len(names)),
                                             batch) for key, t, names, _ in DECODE_LAUNCHES], 4)
    per = {}
    for key, t, names, _ in DECODE_LAUNCHES:
        f = 2.0 * batch * sum(mats[n][1] * mats[n][2] for n in names)
        per[key] = {"avg_us": round(avg[key] * 1e6, 2), "tflops": round(f / avg[key] / 1e12, 1),
                    "frac_of_mfma_peak": round(f / avg[key] / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)}
    dom = max(per, key=lambda k: avg[k])
    fd = 2.0 * batch * sum(mats[n][1] * mats[n][2] for n in dict((k, nm) for k, _, nm, _ in DECODE_LAUNCHES)[dom])
    res = {"us": round(dt * 1e6, 2), "tflops": round(flops / dt / 1e12, 2),
                          "per_launch": per,
                          "roofline": {"bound": "mfma", "achieved": round(fd / avg[dom] / 1e12, 1),
                                       "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                       "frac": round(fd / avg[dom] / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
                                       "traffic": load_traffic("traffic_configs", f"prefill_{dom}"),
                                       "kernel": f"mg_kernel (MFMA dequant-GEMM) {dom} launch",
                                       "flops_per_launch": fd, "avg_launch_us": round(avg[dom] * 1e6, 2),
                                       "timing": TIMING}}
    del copies, arrs, xs, ys
    torch.cuda.empty_cache()
    return res


def bench_llama_singles(torch, np, stream, device, lib, sptr, mats):
    """The layer's distinct matrix shapes alone at batch 1, each over rotated
    copies of more than 600 MB (beyond the 256 MB Infinity Cache)."""
    singles = {}
    for name in ("q", "gate", "down"):
        t, rows, cols, p = mats[name]
        n = max(2, int(np.ceil(600e6 / p.nbytes)))
        first = torch.from_numpy(p).cuda()
        ws1 = [first] + [first.clone() for _ in range(n - 1)]
        x1 = torch.randn(1, cols, device="cuda")
        y1 = torch.empty(1, rows, device="cuda")
        dt = time_graph(torch, stream, [lambda w=w: device.matvec(t, w, x1, rows, cols, out=y1) for w in ws1 * 2])
        arrs1 = [_descs(np, [mats[name]], x1, [y1], [w]) for w in ws1]
        avg1 = timed_grouped(lib, stream, sptr, [(name, t, lambda s: (arrs1[s % len(arrs1)], 1), 1)], 2 * n)[name]
        label = {12: "Q4_K", 14: "Q6_K"}[t]
        singles[f"{name} {rows}x{cols} {label}"] = {
            "us": round(dt * 1e6, 2), "gbs": round(p.nbytes / dt / 1e9, 1),
            "pct_hbm_peak": round(100 * p.nbytes / dt / 1e9 / HBM_PEAK_GBS, 2),
            "roofline": roofline_hbm(p.nbytes, avg1, load_traffic("traffic_configs", f"single_{name}"),
                                     kernel=f"mv_kernel (VALU) {label} batch 1", timing=TIMING)}
        del ws1, first
    return singles


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the other workloads")
    ap.add_argument("--only", default=None,
                    help="run only one workload and print its JSON, for profiling: llama_decode (the headline "
                         "launches, eagerly), q4k_3072x1024, sweep, lm_head_q6k_151936x1024, moe_qwen3_30b_a3b, "
                         "llama3_8b_layer, llama3_8b_prefill, gguf_upload, copy_calibration")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures the dequant-matvec path on one GPU; runs on more than one GPU "
              "are not implemented (--gpus must be 1)", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from pyrite_amd import _lib, device
    from pyrite_amd.quantize import quantize

    lib = _lib.load()
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    # all work goes on one side stream (default priority): graphs cannot be
    # captured on the default stream
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    torch.cuda.set_stream(stream)
    sptr = ctypes.c_void_p(stream.cuda_stream)
    others = {
        "q4k_3072x1024": lambda: bench_q4k_single(torch, np, quantize, lib, stream, sptr, device),
        "sweep": lambda: bench_sweep(torch, np, quantize, lib, stream, sptr, 20),
        "lm_head_q6k_151936x1024": lambda: bench_lm_head(torch, np, quantize, lib, stream, sptr, device),
        "moe_qwen3_30b_a3b": lambda: bench_moe(torch, np, quantize, stream, device),
        "llama3_8b_layer": lambda: bench_llama(torch, np, quantize, stream, device, lib, sptr,
                                               llama_weights(np, quantize)),
        "llama3_8b_prefill": lambda: bench_llama_prefill(torch, np, stream, lib, sptr, llama_weights(np, quantize)),
        "gguf_upload": lambda: bench_gguf_upload(torch, np),
        "copy_calibration": lambda: copy_calibration(torch, stream),
    }
    if args.only and args.only != "llama_decode":
        print(json.dumps({args.only: others[args.only]()}), flush=True)
        return 0

    log("quantizing and uploading the Llama-3-8B layer")
    mats = llama_weights(np, quantize)
    layer_bytes = sum(p.nbytes for _, _, _, p in mats.values())
    copies = [{n: torch.from_numpy(m[3]).cuda() for n, m in mats.items()} for _ in range(DECODE_COPIES)]
    arrs, xs, ys = llama_step_descs(np, torch, mats, 1, copies)

    def step(s: int) -> None:
        run_llama_step(lib, sptr, arrs, 1, s % DECODE_COPIES)

    log(f"warmup {args.warmup} steps; {layer_bytes / 1e6:.1f} MB of quantized weights per step")
    for s in range(args.warmup):
        step(s)
    torch.cuda.synchronize()
    if args.only == "llama_decode":
        for s in range(args.steps):
            step(s)
        torch.cuda.synchronize()
        print(json.dumps({"llama_decode": {"steps": args.steps, "launches": [k for k, *_ in DECODE_LAUNCHES]}}),
              flush=True)
        return 0
    eager_out = {k: v.clone() for k, v in ys.items()}

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for s in range(args.steps):
            step(s)
    g.replay()  # graph warm-up, checked against the eager launches
    torch.cuda.synchronize()
    for k, v in ys.items():
        if not torch.equal(v, eager_out[k]):
            raise RuntimeError(f"graph replay differs from eager launches for {k}")

    log(f"timed: {args.steps} steps in one graph replay")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g.replay()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    value = layer_bytes * args.steps / elapsed / 1e9

    log("per-kernel timing pass")
    avg = timed_grouped(lib, stream, sptr,
                        [(key, t, lambda s, key=key, names=names: (arrs[(key, s % DECODE_COPIES)], len(names)), 1)
                         for key, t, names, _ in DECODE_LAUNCHES], args.steps)
    per_kernel = {}
    for key, t, names, _ in DECODE_LAUNCHES:
        nbytes = sum(mats[n][3].nbytes for n in names)
        per_kernel[key] = {"matrices": "+".join(names), "avg_us": round(avg[key] * 1e6, 3),
                           "total_s": round(avg[key] * args.steps, 9), "bytes_per_launch": nbytes,
                           "gbs": round(nbytes / avg[key] / 1e9, 1),
                           "frac": round(nbytes / avg[key] / 1e9 / HBM_PEAK_GBS, 4)}
    dom = max(per_kernel, key=lambda k: avg[k])
    dnames = per_kernel[dom]["matrices"]
    dtype = {12: "Q4_K", 14: "Q6_K"}[dict((k, t) for k, t, *_ in DECODE_LAUNCHES)[dom]]
    roofline = roofline_hbm(per_kernel[dom]["bytes_per_launch"], avg[dom], load_traffic("traffic_llama_decode", dom),
                            kernel=f"mv_kernel (VALU), the {dom} launch ({dnames}, {dtype}, batch 1)", timing=TIMING)
    del g, copies, arrs, xs, ys
    torch.cuda.empty_cache()

    extra = None
    if not args.no_extra:
        extra = {}
        for name in ("q4k_3072x1024", "sweep", "lm_head_q6k_151936x1024", "moe_qwen3_30b_a3b", "llama3_8b_layer",
                     "gguf_upload"):
            log(f"workload: {name}")
            extra[name] = others[name]()
            torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu_baseline:
        rng = np.random.default_rng(SEED + 7)
        xv = {c: rng.standard_normal(c) for c in (4096, 14336)}
        calls = [(t, p, xv[cols], rows, cols) for t, rows, cols, p in mats.values()]
        what = "the Llama-3-8B layer decode (q, k, v, o, gate, up, down; one vector)"
        log(f"cpu baseline (~{args.cpu_seconds:.0f} s)")
        cpu = run_cpu_baseline(np, calls, args.cpu_seconds, 1, what)
        model, ncpu = cpu_info()
        cpu["host"] = f"{model}, {ncpu} logical CPUs visible"
        nthreads = max(1, min(16, ncpu))  # all host cores (at most 16, the box's CPU share)
        log(f"cpu baseline on {nthreads} threads (~{args.cpu_seconds:.0f} s)")
        cpu["all_cores"] = run_cpu_baseline(np, calls, args.cpu_seconds, nthreads, what)
        del cpu["all_cores"]["kind"]

    moe = (extra or {}).get("moe_qwen3_30b_a3b") or {}
    result = {
        "metric": "dequant-matvec GB/s on quantized bytes (% HBM peak); MoE-layer tokens/s at b=1/64",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded N(0,0.02) fp32 weights quantized by pyrite_amd.quantize, N(0,1) fp32 activations",
        "config": {
            "workload": "Llama-3-8B layer decode, batch 1, Q4_K_M mix: q/o 4096x4096, k/v 1024x4096, "
                        "gate/up 14336x4096 Q4_K, down 4096x14336 Q6_K; four launches per step "
                        "(q/k/v grouped, o, gate/up grouped, down)",
            "bytes_per_step": layer_bytes,
            "weight_copies": DECODE_COPIES,
            "launches_per_step": len(DECODE_LAUNCHES),
        },
        "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "roofline": roofline,
        "moe_tokens_per_s": {b: moe[b]["tokens_per_s"] for b in ("b1", "b64") if b in moe} or None,
        "cpu_baseline": cpu,
        "per_kernel": per_kernel,
        "workloads": extra,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
