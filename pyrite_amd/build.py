"""Build libpyrite_hip.so in-tree with hipcc for gfx950.

    python -m pyrite_amd.build          # compile the csrc/*.hip that changed and link
    python -m pyrite_amd.build --force  # compile every csrc/*.hip

The library lands next to this file (pyrite_amd/libpyrite_hip.so) so that it
travels with the source tree; objects go to pyrite_amd/_build/.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "libpyrite_hip.so"
ARCH = os.environ.get("PYRITE_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops: keep the compiler from emitting v_pk_{add,mul,fma}_f32.
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", str(HERE.parent / "include"),
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build(verbose: bool = False, jobs: int | None = None, force: bool = False) -> Path:
    """Compile and link.  Without ``force`` an object is rebuilt only when it is
    older than its source, any header, or this file (which holds the flags)."""
    BUILD.mkdir(exist_ok=True)
    cc = hipcc()
    srcs = sources()
    headers = list(CSRC.glob("*.h")) + [HERE.parent / "include" / "pyrite_hip.h", Path(__file__).resolve()]
    newest_header = max(p.stat().st_mtime for p in headers)

    def stale(src: Path, obj: Path) -> bool:
        return force or not obj.is_file() or obj.stat().st_mtime < max(src.stat().st_mtime, newest_header)

    def compile_one(src: Path) -> Path:
        obj = BUILD / (src.stem + ".o")
        if not stale(src, obj):
            return obj
        cmd = [cc, *FLAGS, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr[-6000:]}")
        return obj

    n = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    with ThreadPoolExecutor(max_workers=n) as pool:
        objs = list(pool.map(compile_one, srcs))
    if not force and LIB.is_file() and all(LIB.stat().st_mtime >= o.stat().st_mtime for o in objs):
        return LIB
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-4000:]}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    out = build(verbose="-v" in sys.argv, force="--force" in sys.argv)
    print(out)
