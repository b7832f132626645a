"""Build libtagi_hip.so for gfx950 from csrc/*.hip with hipcc.

Each translation unit compiles in its own hipcc process (in parallel), then one hipcc
link produces ``triton_tagi_amd/libtagi_hip.so`` in-tree, next to the Python package
that loads it.

    python triton-tagi_amd/build.py            # build
    python triton-tagi_amd/build.py --jobs 4   # limit parallel compiles
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT_DIR = HERE / "_build"
LIB = HERE / "triton_tagi_amd" / "libtagi_hip.so"
ARCH = "gfx950"

# -packed-fp32-ops off: packed fp32 VALU forms are kept out of every kernel.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}")


def build(jobs: int | None = None, verbose: bool = True) -> Path:
    hipcc = _hipcc()
    OUT_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no sources in {CSRC}")
    objs = [OUT_DIR / (s.stem + ".o") for s in sources]
    jobs = jobs or min(len(sources), max(1, os.cpu_count() or 1))

    def compile_one(pair):
        src, obj = pair
        if verbose:
            print(f"[build] hipcc {src.name}", flush=True)
        _run([hipcc, *HIP_FLAGS, "-c", str(src), "-o", str(obj)])

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(compile_one, zip(sources, objs)))
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, LIB)
    if verbose:
        print(f"[build] wrote {LIB}", flush=True)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args()
    try:
        build(args.jobs)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
