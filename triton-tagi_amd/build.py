"""Build libtagi_hip.so for gfx950 from csrc/*.hip with hipcc.

Each translation unit compiles in its own hipcc process (in parallel; the GEMM kernel
instantiations are split over 18 units), then one hipcc link produces ``triton_tagi_amd/libtagi_hip.so`` in-tree, next to the Python package
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


# tagi_gemm_inst.hip holds the GEMM kernels; it is compiled once per tile config (0..5)
# and product (0..2), each into its own object.
INST = "tagi_gemm_inst.hip"
N_CFG, N_PROD = 6, 3


def compile_units() -> list[tuple[Path, Path, list[str]]]:
    """(source, object, extra defines) for every translation unit."""
    units = []
    for src in sorted(CSRC.glob("*.hip")):
        if src.name == INST:
            for c in range(N_CFG):
                for p in range(N_PROD):
                    units.append((src, OUT_DIR / f"{src.stem}_c{c}_p{p}.o",
                                  [f"-DTAGI_INST_CFG={c}", f"-DTAGI_INST_PROD={p}"]))
        else:
            units.append((src, OUT_DIR / (src.stem + ".o"), []))
    return units


def build(jobs: int | None = None, verbose: bool = True) -> Path:
    hipcc = _hipcc()
    OUT_DIR.mkdir(exist_ok=True)
    units = compile_units()
    if not units:
        raise RuntimeError(f"no sources in {CSRC}")
    objs = [obj for _, obj, _ in units]
    jobs = jobs or min(len(units), max(1, os.cpu_count() or 1))

    def compile_one(unit):
        src, obj, defs = unit
        if verbose:
            print(f"[build] hipcc {src.name} {' '.join(defs)}".rstrip(), flush=True)
        _run([hipcc, *HIP_FLAGS, *defs, "-c", str(src), "-o", str(obj)])

    # the instantiation units are the slowest: start them first
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(compile_one, sorted(units, key=lambda u: not u[2])))
    for stale in OUT_DIR.glob("*.o"):
        if stale not in objs:
            stale.unlink()
    tmp = LIB.with_suffix(".so.tmp")
    # -z defs: a kernel combination missing from the instantiation lists fails here
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs", *map(str, objs), "-o", str(tmp)])
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
