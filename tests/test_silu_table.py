"""CPU check of the build-time bf16 SiLU table (cppvllm_amd.build.write_silu_lut) that the SwiGLU
kernel and the gate/up GEMM epilogues index: every one of the 65536 gate values (NaN, infinities,
subnormals included) equals the CPU oracle's silu (u = 1) bit for bit."""
import numpy as np

from cppvllm_amd import build


def test_silu_table_equals_oracle_for_every_gate(orc, tmp_path):
    path = tmp_path / "silu_bf16_lut.inc"
    build.write_silu_lut(path)
    lut = np.array([int(v, 16) for v in path.read_text().replace(",", " ").split()], dtype=np.uint16)
    assert lut.size == 65536
    g = np.arange(65536, dtype=np.uint32).astype(np.uint16).reshape(64, 1024)
    gu = np.concatenate([g, np.full((64, 1024), 0x3F80, dtype=np.uint16)], axis=1)   # u = 1.0
    want = orc.swiglu(gu, dtype=orc.BF16).reshape(-1)
    bad = np.nonzero(want != lut)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first gate bits 0x{int(bad[0]):04x}"
