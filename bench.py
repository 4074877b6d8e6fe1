#!/usr/bin/env python3
"""Benchmark of the fused GGML dequantize x matvec path on one MI355X.

Workload (the metric's configuration): every Qwen3-0.6B decode projection
(hidden 1024, 16 q / 8 kv heads x head_dim 128: q 2048x1024, k/v 1024x1024,
o 1024x2048, gate/up 3072x1024, down 1024x3072), each quantized from seeded
N(0, 0.02) fp32 weights to Q4_0, Q5_1, Q8_0, Q3_K, Q5_K, Q6_K and IQ4_XS, with
fp32 N(0, 1) activations at batch 1 and 8.

One step = for batch in (1, 8), for each type: one grouped launch
(pyrite_dev_matvec_grouped) over that type's 7 projection matrices.  Weights
are uploaded verbatim and rotated over 4 device copies (305 MB > the 256 MB
Infinity Cache), so every launch reads its weights from HBM.  The timed steps
are captured into one HIP graph and replayed once between two
synchronisations.  Each kernel's duration for the roofline comes from HIP
events that the launch itself records at kernel start and end
(hipExtLaunchKernelGGL), over the same launches replayed eagerly on the same
stream right after the timed replay.

Prints one JSON line.  value = quantized weight bytes / second over the timed
steps (GB/s).  --gpus N > 1 exits: this path runs on one GPU.

The line also carries, under "workloads", the other workloads of the
path, each timed as calls captured in one HIP graph: the single Q4_K
3072x1024 matvec, the Q6_K 151936x1024 LM head with its exact greedy id, the
Qwen3-30B-A3B MoE layer (tokens/s at batch 1, 8, 64) and the Llama-3-8B
Q4_K_M layer (batch-1 decode and 512-token prefill; its q, gate and down
matrices also alone at batch 1), and the GGUF -> HBM upload rate of the
resident-tensor loader.
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


def build_weights(torch, np, quantize):
    """Quantized sweep weights on the device: {type: [(rows, cols, tensor[COPIES])]}."""
    rng = np.random.default_rng(SEED)
    out = {}
    total = 0
    for name, t in SWEEP_TYPES:
        mats = []
        for pname, rows, cols in PROJECTIONS:
            w = (rng.standard_normal(rows * cols, dtype=np.float32) * np.float32(0.02)).astype(np.float64)
            payload = quantize(t, w)
            base = torch.from_numpy(payload).to("cuda")
            copies = [base] + [base.clone() for _ in range(COPIES - 1)]
            mats.append((rows, cols, payload, copies))
            total += payload.nbytes
        out[t] = mats
    return out, total


def run_cpu_baseline(weights, np, budget_s: float):
    """Time the reference's scalar fp64 pyrite_matvec on the host over the sweep."""
    from oracle.oracle import oracle, reference

    impl = reference()
    kind = "reference"
    if impl is None:
        impl = oracle()
        kind = "port"
    rng = np.random.default_rng(SEED + 7)
    xs = {cols: rng.standard_normal((8, cols)) for cols in {c for _, _, c in PROJECTIONS}}
    done_bytes = 0
    passes = 0
    t0 = time.perf_counter()
    while True:
        for _, t in SWEEP_TYPES:
            for rows, cols, payload, _ in weights[t]:
                for batch in BATCHES:
                    for b in range(batch):
                        impl.matvec(t, payload, xs[cols][b], rows, cols)
                        done_bytes += payload.nbytes
        passes += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    dt = time.perf_counter() - t0
    return {"value": done_bytes / dt / 1e9, "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": f"{passes} pass(es) of the full sweep (7 types x 7 projections, batch 1 and 8 as 1+8 "
                      f"single-vector calls) through pyrite_matvec, single thread, {dt:.1f} s"}


def run_cpu_baseline_parallel(weights, np, budget_s: float, nthreads: int):
    """The same sweep on all host cores: thread i runs every call of the sweep
    on its own contiguous i-th share of each matrix's rows (the reference
    function is reentrant and rows are independent), so the threads never
    wait for each other; throughput = all threads' bytes over the wall time."""
    import threading

    from oracle.oracle import oracle, reference

    impl = reference() or oracle()
    rng = np.random.default_rng(SEED + 7)
    xs = {cols: rng.standard_normal((8, cols)) for cols in {c for _, _, c in PROJECTIONS}}
    calls = []
    for _, t in SWEEP_TYPES:
        for rows, cols, payload, _ in weights[t]:
            rb = payload.nbytes // rows
            for batch in BATCHES:
                for b in range(batch):
                    calls.append((t, payload, rb, xs[cols][b], rows, cols))
    done = [0] * nthreads
    passes = [0] * nthreads
    errors = []
    start = threading.Barrier(nthreads + 1)
    deadline = [0.0]

    def worker(i):
        outs = {}
        start.wait()
        while True:
            for t, payload, rb, x, rows, cols in calls:
                r0, r1 = rows * i // nthreads, rows * (i + 1) // nthreads
                if r1 <= r0:
                    continue
                out = outs.setdefault((rows, r1 - r0), np.zeros(r1 - r0, dtype=np.float64))
                if impl.matvec_raw(t, payload[r0 * rb:r1 * rb], x, out, r1 - r0, cols) != 0:
                    errors.append(t)
                    return
                done[i] += (r1 - r0) * rb
            passes[i] += 1
            if time.perf_counter() >= deadline[0]:
                return

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(nthreads)]
    for th in threads:
        th.start()
    t0 = time.perf_counter()
    deadline[0] = t0 + budget_s
    start.wait()
    for th in threads:
        th.join()
    dt = time.perf_counter() - t0
    if errors:
        raise ValueError("pyrite_matvec failed")
    return {"value": sum(done) / dt / 1e9, "unit": "GB/s", "cores": nthreads,
            "sample": f"{min(passes)}-{max(passes)} pass(es) of the same sweep per thread, thread i on its "
                      f"i-th share of every matrix's rows, {nthreads} threads, {dt:.1f} s"}


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
    """Kernel that pyrite_dev_matvec_grouped runs for this type and batch (block formats)."""
    return "mx_kernel (MFMA)" if batch >= 3 else "mv_kernel (VALU)"


def load_traffic(key: str):
    """HBM bytes per launch of a sweep launch ("<type>_b<batch>") from the committed
    FETCH_SIZE / WRITE_SIZE profile (profiles/traffic_sweep.json), or None."""
    path = ROOT / "profiles" / "traffic_sweep.json"
    try:
        data = json.loads(path.read_text())
    except (OSError, ValueError):
        return None
    entry = data.get("launches", {}).get(key)
    return None if entry is None else entry.get("hbm_bytes_per_launch")


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


def bench_q4k_single(torch, np, quantize, stream, device):
    """Single Q4_K 3072x1024 matvec (Qwen3-0.6B ffn_up), batch 1."""
    rows, cols = 3072, 1024
    p = quantized_normal(np, quantize, 12, rows * cols, SEED + 11)
    ws = [torch.from_numpy(p).cuda() for _ in range(160)]  # 283 MB of copies
    x = torch.randn(1, cols, device="cuda")
    y = torch.empty(1, rows, device="cuda")
    calls = [lambda w=w: device.matvec(12, w, x, rows, cols, out=y) for w in ws]
    dt = time_graph(torch, stream, calls)
    return {"workload": "Q4_K 3072x1024 matvec, batch 1", "us": round(dt * 1e6, 3),
            "gbs": round(p.nbytes / dt / 1e9, 1), "pct_hbm_peak": round(100 * p.nbytes / dt / 1e9 / HBM_PEAK_GBS, 2)}


def bench_lm_head(torch, np, quantize, stream, device):
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
    return {"workload": "Q6_K 151936x1024 LM head, batch 1 (logits + exact greedy id)",
            "us_per_token": round(dt_head * 1e6, 2), "tokens_per_s": round(1 / dt_head, 1),
            "gbs": round(p.nbytes / dt_head / 1e9, 1),
            "pct_hbm_peak": round(100 * p.nbytes / dt_head / 1e9 / HBM_PEAK_GBS, 2),
            "matvec_only_us": round(dt_mv * 1e6, 2), "matvec_only_gbs": round(p.nbytes / dt_mv / 1e9, 1),
            "bytes_per_token": p.nbytes}


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
                            "pct_hbm_peak": round(100 * nbytes / dt / 1e9 / HBM_PEAK_GBS, 2)}
    out["workload"] = ("Qwen3-30B-A3B MoE FFN layer: router F32 2048x128, gate/up Q4_K [128x768x2048], "
                       f"down Q6_K [128x2048x768], top-8, renormalised; {distinct_experts} seeded quantized "
                       "experts tiled over the 128 slices, 2 layer copies alternated, distinct inputs per call")
    return out


def bench_llama(torch, np, quantize, stream, device, lib, sptr):
    """Llama-3-8B layer in Q4_K_M mix: decode (batch 1) and 512-token prefill."""
    shapes = [("q", 12, 4096, 4096), ("k", 12, 1024, 4096), ("v", 12, 1024, 4096), ("o", 12, 4096, 4096),
              ("gate", 12, 14336, 4096), ("up", 12, 14336, 4096), ("down", 14, 4096, 14336)]
    cache = {}
    mats = []
    for name, t, rows, cols in shapes:
        key = (t, rows, cols)
        if key not in cache:
            cache[key] = quantized_normal(np, quantize, t, rows * cols, SEED + 20 + len(cache))
        mats.append((name, t, rows, cols, cache[key]))
    layer_bytes = sum(m[4].nbytes for m in mats)
    copies = 3
    dev = [[torch.from_numpy(m[4]).cuda() for m in mats] for _ in range(copies)]
    res = {"workload": "Llama-3-8B layer, Q4_K_M mix: q/o 4096x4096, k/v 1024x4096, gate/up 14336x4096 Q4_K, "
                       "down 4096x14336 Q6_K", "bytes_per_layer": layer_bytes}
    for batch, reps in ((1, 12), (512, 2)):
        xs = {c: torch.randn(batch, c, device="cuda") for c in (4096, 14336)}
        ys = [torch.empty(batch, m[2], device="cuda") for m in mats]

        def layer(i):
            ws = dev[i % copies]
            q4 = [j for j, m in enumerate(mats) if m[1] == 12]
            arr = (Desc * len(q4))()
            for a, j in enumerate(q4):
                _, t, rows, cols, p = mats[j]
                arr[a] = Desc(ws[j].data_ptr(), p.nbytes, rows, cols, xs[cols].data_ptr(), cols, ys[j].data_ptr(), rows)
            rc = lib.pyrite_dev_matvec_grouped(12, arr, len(q4), batch, sptr)
            if rc != 0:
                raise RuntimeError(f"grouped matvec failed: {rc} {lib.pyrite_hip_last_error()}")
            j = len(mats) - 1
            device.matvec(14, ws[j], xs[14336], mats[j][2], mats[j][3], out=ys[j])
        dt = time_graph(torch, stream, [lambda i=i: layer(i) for i in range(reps)])
        flops = 2.0 * batch * sum(m[2] * m[3] for m in mats)
        key = "decode_b1" if batch == 1 else "prefill_512"
        res[key] = {"us": round(dt * 1e6, 2), "gbs": round(layer_bytes / dt / 1e9, 1),
                    "pct_hbm_peak": round(100 * layer_bytes / dt / 1e9 / HBM_PEAK_GBS, 2),
                    "tflops": round(flops / dt / 1e12, 2)}
    del dev
    # The layer's distinct matrix shapes alone at batch 1, each over rotated
    # copies of more than 600 MB (beyond the 256 MB Infinity Cache).
    singles = {}
    for name, t, rows, cols, p in mats:
        if name not in ("q", "gate", "down"):
            continue
        n = max(2, int(np.ceil(600e6 / p.nbytes)))
        first = torch.from_numpy(p).cuda()
        ws1 = [first] + [first.clone() for _ in range(n - 1)]
        x1 = torch.randn(1, cols, device="cuda")
        y1 = torch.empty(1, rows, device="cuda")
        dt = time_graph(torch, stream, [lambda w=w: device.matvec(t, w, x1, rows, cols, out=y1) for w in ws1 * 2])
        label = {12: "Q4_K", 14: "Q6_K"}[t]
        singles[f"{name} {rows}x{cols} {label}"] = {
            "us": round(dt * 1e6, 2), "gbs": round(p.nbytes / dt / 1e9, 1),
            "pct_hbm_peak": round(100 * p.nbytes / dt / 1e9 / HBM_PEAK_GBS, 2)}
        del ws1, first
    res["decode_b1_matrices"] = singles
    return res


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the LM-head, MoE and Llama configurations")
    ap.add_argument("--only", default=None,
                    help="run only the named extra configuration (q4k_3072x1024, lm_head_q6k_151936x1024, "
                         "moe_qwen3_30b_a3b, llama3_8b_layer, gguf_upload, copy_calibration) and print its JSON; "
                         "for profiling")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures the dequant-matvec path on one GPU; runs on more than one GPU "
              "are not implemented (--gpus must be 1)", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from pyrite_amd import _lib
    from pyrite_amd.quantize import quantize

    lib = _lib.load()
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    if args.only:
        from pyrite_amd import device
        stream = torch.cuda.Stream()
        torch.cuda.set_stream(stream)
        sptr = ctypes.c_void_p(stream.cuda_stream)
        fns = {"q4k_3072x1024": lambda: bench_q4k_single(torch, np, quantize, stream, device),
               "lm_head_q6k_151936x1024": lambda: bench_lm_head(torch, np, quantize, stream, device),
               "moe_qwen3_30b_a3b": lambda: bench_moe(torch, np, quantize, stream, device),
               "llama3_8b_layer": lambda: bench_llama(torch, np, quantize, stream, device, lib, sptr),
               "gguf_upload": lambda: bench_gguf_upload(torch, np),
               "copy_calibration": lambda: copy_calibration(torch, stream)}
        print(json.dumps({args.only: fns[args.only]()}), flush=True)
        return 0
    log("quantizing and uploading the sweep weights")
    weights, bytes_per_set = build_weights(torch, np, quantize)
    rng = np.random.default_rng(SEED + 1)
    xs = {(cols, b): torch.from_numpy(rng.standard_normal((b, cols), dtype=np.float32)).cuda()
          for cols in {c for _, _, c in PROJECTIONS} for b in BATCHES}
    ys = {(t, i, b): torch.empty(b, rows, dtype=torch.float32, device="cuda")
          for _, t in SWEEP_TYPES for i, (_, rows, _c) in enumerate(PROJECTIONS) for b in BATCHES}

    descs = {}
    for _, t in SWEEP_TYPES:
        for b in BATCHES:
            for c in range(COPIES):
                arr = (Desc * len(PROJECTIONS))()
                for i, (rows, cols, payload, copies) in enumerate(weights[t]):
                    x = xs[(cols, b)]
                    y = ys[(t, i, b)]
                    arr[i] = Desc(copies[c].data_ptr(), payload.nbytes, rows, cols, x.data_ptr(), cols,
                                  y.data_ptr(), rows)
                descs[(t, b, c)] = arr
    # all work goes on one side stream (default priority): graphs cannot be
    # captured on the default stream
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    torch.cuda.set_stream(stream)
    sptr = ctypes.c_void_p(stream.cuda_stream)
    fn = lib.pyrite_dev_matvec_grouped

    launches = [(t, b) for b in BATCHES for _, t in SWEEP_TYPES]

    def step(s: int, events=None) -> None:
        for k, (t, b) in enumerate(launches):
            c = (2 * s + BATCHES.index(b)) % COPIES
            if events is not None:
                events[k][0].record(stream)
            rc = fn(t, descs[(t, b, c)], len(PROJECTIONS), b, sptr)
            if rc != 0:
                raise RuntimeError(f"pyrite_dev_matvec_grouped({t}, batch {b}) returned {rc}: {_lib.last_error()}")
            if events is not None:
                events[k][1].record(stream)

    bytes_per_step = bytes_per_set * len(BATCHES)
    log(f"warmup {args.warmup} steps; {bytes_per_step / 1e6:.1f} MB of quantized weights per step")
    for s in range(args.warmup):
        step(s)
    torch.cuda.synchronize()
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
    value = bytes_per_step * args.steps / elapsed / 1e9

    # Per-kernel durations: the same launches again, eagerly, each timed by HIP
    # events that the launch itself records at kernel start and end
    # (pyrite_dev_matvec_grouped_timed -> hipExtLaunchKernelGGL), on this stream.
    log("per-kernel timing pass")
    timed = lib.pyrite_dev_matvec_grouped_timed
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in launches]
    for pair in evs:
        for e in pair:
            e.record(stream)  # creates the underlying hipEvent_t
    torch.cuda.synchronize()
    durations = {}
    for s in range(args.steps):
        for k, (t, b) in enumerate(launches):
            c = (2 * s + BATCHES.index(b)) % COPIES
            rc = timed(t, descs[(t, b, c)], len(PROJECTIONS), b, sptr, ctypes.c_void_p(evs[k][0].cuda_event),
                       ctypes.c_void_p(evs[k][1].cuda_event))
            if rc != 0:
                raise RuntimeError(f"timed launch failed: {rc} {_lib.last_error()}")
        torch.cuda.synchronize()
        for k, key in enumerate(launches):
            durations.setdefault(key, []).append(evs[k][0].elapsed_time(evs[k][1]) * 1e-3)
    timing_source = ("HIP events recorded by each launch at kernel start/end (hipExtLaunchKernelGGL), "
                     "same launches and weight rotation as the timed graph, on the same stream")

    per_kernel = {}
    for (t, b), ds in durations.items():
        name = dict((v, n) for n, v in SWEEP_TYPES)[t]
        nbytes = sum(p.nbytes for _, _, p, _ in weights[t])
        avg = sum(ds) / len(ds)
        per_kernel[f"{name}_b{b}"] = {"avg_us": avg * 1e6, "total_s": sum(ds), "bytes_per_launch": nbytes,
                                      "gbs": nbytes / avg / 1e9}
    dominant = max(per_kernel, key=lambda k: per_kernel[k]["total_s"])
    dk = per_kernel[dominant]
    dom_batch = int(dominant.rsplit("_b", 1)[1])
    roofline = {"bound": "hbm", "achieved": round(dk["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(dk["gbs"] / HBM_PEAK_GBS, 4), "traffic": load_traffic(dominant),
                "kernel": f"{launch_kernel_name(dom_batch)} {dominant} (grouped launch over the 7 projections)",
                "avg_launch_us": round(dk["avg_us"], 3), "bytes_per_launch": dk["bytes_per_launch"],
                "timing": timing_source}

    extra = None
    if not args.no_extra:
        from pyrite_amd import device
        extra = {}
        for name, fn in (("q4k_3072x1024", lambda: bench_q4k_single(torch, np, quantize, stream, device)),
                         ("lm_head_q6k_151936x1024", lambda: bench_lm_head(torch, np, quantize, stream, device)),
                         ("moe_qwen3_30b_a3b", lambda: bench_moe(torch, np, quantize, stream, device)),
                         ("llama3_8b_layer", lambda: bench_llama(torch, np, quantize, stream, device, lib,
                                                                         sptr)),
                         ("gguf_upload", lambda: bench_gguf_upload(torch, np))):
            log(f"extra configuration: {name}")
            extra[name] = fn()
            torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu_baseline:
        log(f"cpu baseline (~{args.cpu_seconds:.0f} s)")
        cpu = run_cpu_baseline(weights, np, args.cpu_seconds)
        model, ncpu = cpu_info()
        cpu["host"] = f"{model}, {ncpu} logical CPUs visible"
        # all host cores (at most 16, the box's CPU share)
        nthreads = max(1, min(16, ncpu))
        log(f"cpu baseline on {nthreads} threads (~{args.cpu_seconds:.0f} s)")
        cpu["all_cores"] = run_cpu_baseline_parallel(weights, np, args.cpu_seconds, nthreads)

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
            "workload": "Qwen3-0.6B decode projection type sweep: q 2048x1024, k/v 1024x1024, o 1024x2048, "
                        "gate/up 3072x1024, down 1024x3072 x {Q4_0,Q5_1,Q8_0,Q3_K,Q5_K,Q6_K,IQ4_XS} x batch {1,8}",
            "bytes_per_step": bytes_per_step,
            "weight_copies": COPIES,
            "launches_per_step": len(launches),
        },
        "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "workloads": extra,
        "per_kernel": {k: {kk: round(vv, 3) if isinstance(vv, float) else vv for kk, vv in v.items()}
                       for k, v in sorted(per_kernel.items())},
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
