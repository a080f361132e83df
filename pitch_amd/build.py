"""Builds libpitch_amd.so in-tree: hipcc for gfx950, one object per per-vector dimension, in parallel.

    python -m pitch_amd.build        # or pitch_amd.build.build()

Steps: generate csrc/pitch_tables.inc from data/codebooks.json, compile csrc/pitch_vector.hip once per
dimension and element type of the uncompressed vectors (-DPITCH_DIM=2..1024, -DPITCH_IO=0/1/2 for
float32/float16/bfloat16), csrc/pitch_channel.hip once per element type, csrc/pitch_attention.hip once per
attention dimension (64, 128) and csrc/pitch_abi.cpp, and link the shared library next to this file. Object files go to <repo>/_build/.
Also builds libpitch_calib.so from csrc/pitch_calib.hip: the measurement kernels bench.py times beside the
codec (not part of the codec's C ABI).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
REPO = PKG.parent
BUILD = REPO / "_build"
LIB = PKG / "libpitch_amd.so"
CALIB_LIB = PKG / "libpitch_calib.so"
DIMS = [2 ** k for k in range(1, 11)]
IO_TYPES = [0, 1, 2]   # element type of uncompressed vectors: float32, float16, bfloat16
ATTENTION_DIMS = [64, 128]
ARCH = os.environ.get("PITCH_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",                           # no implicit FMA: the reference's roundings are kept
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{CSRC}",
]


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found: install ROCm or put hipcc on PATH")
    return exe


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compiles every source and links LIB. Always rebuilds."""
    hipcc = _hipcc()
    BUILD.mkdir(exist_ok=True)
    _run([sys.executable, str(CSRC / "gen_tables.py"), str(PKG / "data" / "codebooks.json"),
          str(CSRC / "pitch_tables.inc")])
    units = [(CSRC / "pitch_vector.hip", BUILD / f"vector_d{d}_io{io}.o", [f"-DPITCH_DIM={d}", f"-DPITCH_IO={io}"], d)
             for d in DIMS for io in IO_TYPES]
    units += [(CSRC / "pitch_channel.hip", BUILD / f"channel_io{io}.o", [f"-DPITCH_IO={io}"], 512) for io in IO_TYPES]
    units += [(CSRC / "pitch_attention.hip", BUILD / f"attention_d{d}.o", [f"-DPITCH_DIM={d}"], 2048 + d)
              for d in ATTENTION_DIMS]
    units += [(CSRC / "pitch_abi.cpp", BUILD / "abi.o", [], 0)]
    # largest dims first: they take longest to compile
    units.sort(key=lambda u: -u[3])
    jobs = jobs or min(8, os.cpu_count() or 4)

    def compile_one(u):
        src, obj, extra, _ = u
        cmd = [hipcc, *HIPCC_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        _run(cmd)
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, units))
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, LIB)
    tmp = CALIB_LIB.with_suffix(".so.tmp")
    _run([hipcc, *HIPCC_FLAGS, "-shared", str(CSRC / "pitch_calib.hip"), "-o", str(tmp)])
    os.replace(tmp, CALIB_LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
