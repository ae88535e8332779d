"""Build the gfx950 HIP library ``cppvllm_amd/libcppvllm_hip.so`` in-tree with hipcc.

Usage: ``python -m cppvllm_amd.build`` (or ``build()`` from Python). Cross-compiles for gfx950
on a machine without a GPU. Every call recompiles.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libcppvllm_hip.so"
OBJ_DIR = PKG / "_build"

# Common device flags. Packed FP32 instructions are disabled on purpose (the device pass
# honours the feature; the host pass warns that it does not know it, which is harmless).
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

# Per-source extra flags. The fused ops are bit-exact against the CPU oracle, so no FMA
# contraction is allowed there; sqrt and division stay correctly rounded (hipcc default).
SOURCES = {
    "fused_ops.hip": ["-ffp-contract=off"],
    "paged_attention.hip": [],
    "paged_prefill.hip": [],
    "gemm.hip": ["-ffp-contract=off"],
    "batch_metadata.hip": ["-ffp-contract=off"],
    "model_ops.hip": ["-ffp-contract=off"],
}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    return "hipcc"


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}")
    for line in (proc.stdout + proc.stderr).splitlines():
        if "packed-fp32-ops" in line or "ignoring feature" in line or not line.strip():
            continue
        sys.stderr.write(line + "\n")


ENGINE_LIB = PKG / "libcvh_engine.so"
ENGINE_SOURCES = ["engine_core.cpp"]


def build_engine(verbose: bool = False) -> Path:
    """Compile the host-only serving core (scheduler, block manager) with g++."""
    tmp = ENGINE_LIB.with_suffix(".so.tmp")
    cmd = [os.environ.get("CXX", "g++"), "-std=c++17", "-O2", "-Wall", "-Wextra", "-fPIC", "-shared", "-o", str(tmp),
           *[str(CSRC / s) for s in ENGINE_SOURCES]]
    if verbose:
        print(" ".join(cmd))
    _run(cmd)
    os.replace(tmp, ENGINE_LIB)
    return ENGINE_LIB


def build(verbose: bool = False) -> Path:
    """Compile every HIP source for gfx950 and link the shared library (and the host serving
    core). Returns the HIP library's path."""
    build_engine(verbose)
    hipcc = _hipcc()
    OBJ_DIR.mkdir(exist_ok=True)
    objs, cmds = [], []
    for src, extra in SOURCES.items():
        obj = OBJ_DIR / (Path(src).stem + ".o")
        cmds.append([hipcc, *HIPCC_FLAGS, *extra, "-c", str(CSRC / src), "-o", str(obj)])
        objs.append(str(obj))
        if verbose:
            print(" ".join(cmds[-1]))
    # one hipcc per source, in parallel (each is single-threaded)
    with ThreadPoolExecutor(max_workers=min(len(cmds), os.cpu_count() or 1)) as pool:
        list(pool.map(_run, cmds))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *objs]
    if verbose:
        print(" ".join(cmd))
    _run(cmd)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
