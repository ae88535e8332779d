"""The libtorch binding shown to maintainers compiles against torch's headers and include/cppvllm_hip.h.

The C++ blocks of the maintainer-facing integration guide at the repository root are the shims
that replace the reference's kernel entry points (kernels/paged_attention.h:5-7,
kernels/fused_ops.h:7-22) and the linear/SwiGLU call sites (model/model_architecture.cpp:155,
178-185). A syntax-only compile keeps their signatures in step with the header. Skipped where g++ or torch's C++ headers are absent.
"""
import re
import shutil
import subprocess
import textwrap
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
GUIDE = "INTEGRATION.md"


def _torch_include():
    import torch
    inc = Path(torch.__file__).parent / "include"
    return inc if (inc / "c10" / "hip" / "HIPStream.h").exists() else None


def test_integration_shims_compile(tmp_path):
    gxx = shutil.which("g++")
    inc = _torch_include()
    if gxx is None or inc is None:
        pytest.skip("g++ or torch's ROCm C++ headers not available")
    text = (ROOT / GUIDE).read_text()
    blocks = re.findall(r"```cpp\n(.*?)```", text, re.S)
    assert len(blocks) >= 2, "the integration guide lost its C++ binding blocks"
    src = tmp_path / "hip_kernels.cpp"
    src.write_text("#include <algorithm>\n" + "\n".join(textwrap.dedent(b) for b in blocks))
    cmd = [gxx, "-std=c++17", "-fsyntax-only", "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM",
           f"-I{inc}", f"-I{inc / 'torch' / 'csrc' / 'api' / 'include'}", "-I/opt/rocm/include",
           f"-I{ROOT / 'include'}", str(src)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr[-4000:]
