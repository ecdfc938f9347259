"""Build the gfx950 library: every csrc/*.hip into libuor_gfx950.so, in-tree.

Run as `python uor-matmul_amd/build.py`; __graft_entry__.build() calls main().
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import pathlib
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT = HERE / "libuor_gfx950.so"
OBJ = HERE / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall",
    # Packed fp32 VALU forms are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _compile(src: pathlib.Path) -> pathlib.Path:
    obj = OBJ / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def main() -> pathlib.Path:
    OBJ.mkdir(exist_ok=True)
    # The residue-number-system constants of the exact float route.
    subprocess.run([sys.executable, str(CSRC / "gen_crt_tables.py")], check=True)
    srcs = sorted(CSRC.glob("*.hip"))
    workers = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=max(1, workers)) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = OUT.with_suffix(".so.tmp")
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs),
                    "-o", str(tmp)], check=True)
    os.replace(tmp, OUT)
    build_probe()
    return OUT


PROBE_SRC = HERE / "probe" / "peaks.hip"
PROBE_OUT = HERE / "libuor_probe.so"


def build_probe() -> pathlib.Path:
    """The calibration probes bench.py runs beside the library (measured HBM
    read and int8 MFMA peaks); a library of their own."""
    tmp = PROBE_OUT.with_suffix(".so.tmp")
    r = subprocess.run([HIPCC, *FLAGS, "-shared", str(PROBE_SRC), "-o", str(tmp)],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {PROBE_SRC.name}:\n{r.stderr}")
    os.replace(tmp, PROBE_OUT)
    return PROBE_OUT


if __name__ == "__main__":
    print(main())
