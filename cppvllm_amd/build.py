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
    "decode_runner.cpp": [],
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


SILU_LUT = OBJ_DIR / "silu_bf16_lut.inc"


def write_silu_lut(path: Path = SILU_LUT) -> None:
    """The bf16 SiLU table the kernels index by a gate's 16 bits: silu(g) = g / (1 + exp(-g))
    in double (the reference's formula, kernels/fused_ops.cu:210-219; exp from the C library,
    IEEE double division), converted to float, then rounded to bf16 (nearest even; NaN -> quiet
    NaN with its sign). Generated at build time into the object directory."""
    import math

    import numpy as np
    bits = np.arange(65536, dtype=np.uint32)
    with np.errstate(all="ignore"):
        g = (bits << 16).view(np.float32).astype(np.float64)

    def c_exp(x: float) -> float:
        if math.isnan(x):
            return x
        try:
            return math.exp(x)
        except OverflowError:
            return math.inf
    e = np.array([c_exp(-x) for x in g.tolist()], dtype=np.float64)
    with np.errstate(all="ignore"):
        s = np.where(np.isnan(g), g, g / (1.0 + e)).astype(np.float32)
    u = s.view(np.uint32)
    rne = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    out = np.where((u & 0x7FFFFFFF) > 0x7F800000, (u >> 16) | 0x40, rne).astype(np.uint32)
    path.parent.mkdir(exist_ok=True)
    lines = [", ".join(f"0x{int(v):04x}" for v in out[i:i + 16]) + "," for i in range(0, 65536, 16)]
    tmp = path.with_suffix(".tmp")
    tmp.write_text("\n".join(lines) + "\n")
    os.replace(tmp, path)


def build(verbose: bool = False) -> Path:
    """Compile every HIP source for gfx950 and link the shared library (and the host serving
    core). Returns the HIP library's path."""
    build_engine(verbose)
    hipcc = _hipcc()
    OBJ_DIR.mkdir(exist_ok=True)
    write_silu_lut()
    objs, cmds = [], []
    for src, extra in SOURCES.items():
        obj = OBJ_DIR / (Path(src).stem + ".o")
        cmds.append([hipcc, *HIPCC_FLAGS, *extra, f"-I{OBJ_DIR}", "-c", str(CSRC / src), "-o", str(obj)])
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
