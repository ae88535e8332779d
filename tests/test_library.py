"""CPU checks of the C ABI library: it loads without a GPU, exports every symbol the header
declares, validates arguments before touching the device, and sizes workspaces consistently.
Plus host-side workload generators and byte accounting."""
import ctypes as C

import pytest
import torch

from cppvllm_amd import _lib, workloads


def test_library_exports_every_header_symbol():
    lib = _lib.lib()
    names = _lib.header_symbols()
    assert len(names) >= 13
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES), "ctypes signature table out of sync with the header"
    assert b"gfx950" in lib.cvh_version()


@pytest.mark.skipif(torch.cuda.is_available(), reason="passes dummy device pointers; CPU-only check")
def test_argument_validation_without_device():
    # Every call below must be rejected (or be a T == 0 no-op) before any kernel launch.
    lib = _lib.lib()
    ok, bad, unsup = _lib.CVH_OK, _lib.CVH_ERR_INVALID_ARG, _lib.CVH_ERR_UNSUPPORTED
    # T == 0 is a no-op success; null pointers are rejected before any device call
    assert lib.cvh_paged_attention_fp8(*[None] * 7, 1, None, None, 0, 16, 8, 128, 16, 0, 0.1, None, 0, None) == ok
    assert lib.cvh_paged_attention_fp8(*[None] * 7, 1, None, None, 4, 16, 8, 128, 16, 0, 0.1, None, 0, None) == bad
    assert lib.cvh_rms_norm(None, None, None, 0, 1024, 1e-6, 0, None) == ok
    assert lib.cvh_rms_norm(None, None, None, 3, 1024, 1e-6, 0, None) == bad
    assert lib.cvh_add_rms_norm(None, None, None, None, -1, 1024, 1e-6, 0, None) == bad
    assert lib.cvh_qk_norm_rope_kv_write_fp8(*[None] * 14, 0, 16, 8, 128, 16, 0, 1e-6, None) == ok
    assert lib.cvh_build_token_metadata(None, 0, None, 0, None, 0, 16, None, None, None, None) == ok
    # unsupported shapes are reported as such (dummy non-null pointers, never dereferenced)
    p = C.c_void_p(16)
    args = [p] * 7
    assert lib.cvh_paged_attention_fp8(*args, 4, p, p, 4, 16, 8, 96, 16, 0, 0.1, None, 0, None) == unsup
    assert lib.cvh_paged_attention_fp8(*args, 4, p, p, 4, 24, 8, 128, 16, 0, 0.1, None, 0, None) == unsup
    assert lib.cvh_paged_attention_fp8(*args, 4, p, p, 4, 16, 8, 128, 24, 0, 0.1, None, 0, None) == unsup
    assert lib.cvh_paged_attention_fp8(*args, 4, p, p, 4, 16, 8, 128, 8, 0, 0.1, None, 0, None) == unsup
    assert lib.cvh_paged_attention_fp8_ex(*args, 4, p, p, 4, 16, 8, 128, 16, 0, 0.1, -3, None, 0, None) == bad
    # the plan needs only the metadata pointers and a workspace
    assert lib.cvh_paged_attention_plan(None, 4, p, p, 4, 16, 8, 128, 16, 0, p, 1 << 30, None) == bad
    assert lib.cvh_paged_attention_plan(p, 4, p, p, 4, 16, 8, 128, 16, 0, None, 0, None) == _lib.CVH_ERR_WORKSPACE
    assert lib.cvh_paged_attention_fp8_planned(*args, 4, p, p, 4, 16, 8, 96, 16, 0, 0.1, 0, p, 1 << 30,
                                               None) == unsup
    # workspace missing
    assert lib.cvh_paged_attention_fp8_ex(*args, 8, p, p, 4, 16, 8, 128, 16, 0, 0.1, 64, None, 0,
                                          None) == _lib.CVH_ERR_WORKSPACE
    # too many rows for one launch: 8192 tokens at <= 8 kv heads, 4096 at 16
    assert lib.cvh_paged_attention_fp8(*args, 1, p, p, 20000, 16, 8, 128, 16, 0, 0.1, p, 1 << 30,
                                       None) == unsup
    assert lib.cvh_paged_attention_fp8(*args, 1, p, p, 8193, 16, 8, 128, 16, 0, 0.1, p, 1 << 30,
                                       None) == unsup
    assert lib.cvh_paged_attention_fp8(*args, 1, p, p, 8193, 4, 4, 128, 16, 0, 0.1, p, 1 << 30,
                                       None) == unsup
    assert lib.cvh_paged_attention_fp8(*args, 1, p, p, 4097, 16, 16, 128, 16, 0, 0.1, p, 1 << 30,
                                       None) == unsup
    assert lib.cvh_rms_norm(p, p, p, 3, 1020, 1e-6, 0, None) == unsup
    assert lib.cvh_rms_norm(p, p, p, 3, 1024, 1e-6, 7, None) == unsup
    assert lib.cvh_qk_norm_rope_kv_write_fp8(*[p] * 14, 4, 16, 8, 96, 16, 0, 1e-6, None) == unsup
    assert lib.cvh_qk_norm_rope_kv_write_fp8(*[p] * 14, 4, 16, 8, 128, 20, 0, 1e-6, None) == unsup


def test_partition_policy_and_workspace_sizes():
    lib = _lib.lib()
    # headline decode (256 tokens, 8 kv heads = one 8-wave row group, 8 x 256-token blocks):
    # 256 partitions (2048 resident waves / 8)
    assert lib.cvh_paged_attention_partitions(256, 8, 8, 256) == 256
    rows, slots = 256, 256 * 2 * 16     # [G][2][WPG*REP] partial slots
    r256 = lambda v: (v + 255) // 256 * 256
    # plan: int2 token metadata [T] + int32 shared-prefix keys [T] + 64-byte workgroup records [G]
    want = r256((rows + 1) * 4) + r256(slots * 128 * 4) + r256(slots * 2 * 4) + r256(256 * 8) + r256(256 * 4) + \
        r256(256 * 64)
    assert lib.cvh_paged_attention_workspace_bytes(256, 16, 8, 128, 8, 256, 0) == want
    # small batches: never less than two tiles per partition
    assert lib.cvh_paged_attention_partitions(1, 1, 1, 16) == 1
    assert lib.cvh_paged_attention_partitions(8, 8, 4, 256) == 8 * 32 // 2
    assert lib.cvh_paged_attention_workspace_bytes(4, 16, 8, 128, 8, 16, -1) == 0


def test_rope_tables_reject_bad_args():
    assert _lib.lib().cvh_rope_tables_host(None, None, 4, 128, 1e6) == _lib.CVH_ERR_INVALID_ARG


def test_workload_generators_shapes():
    b = workloads.config1(device="cpu")
    assert b["q"].shape == (8, 16, 128) and b["k_cache"].shape[1:] == (256, 8, 128)
    assert b["k_scale"].numel() == 1 and b["num_blocks"] == 64
    lens = b["token_kv_len"].tolist()
    assert all(100 <= L <= 1024 for L in lens)
    t = b["block_tables"]
    used = t[t >= 0]
    assert used.unique().numel() == used.numel()          # distinct blocks across sequences
    lens3 = workloads.config3_lens()
    assert len(lens3) == 256 and all(100 <= L <= 2048 for L in lens3)
    lens4 = workloads.config4_lens()
    assert all(4096 <= L <= 32768 for L in lens4)
    f = workloads.fused_batch(T=512, n_segments=8)
    assert (f["slots"][f["valid_tokens"]:] == -1).all()
    s = f["slots"][:f["valid_tokens"]]
    assert s.unique().numel() == s.numel() and (s >= 0).all()


def test_quantize_blocks_layout():
    x = torch.randn(2, 16, 8, 128)
    codes, sc = workloads.quantize_blocks(x, per_tensor=False)
    assert codes.dtype == torch.uint8 and sc.shape == (2, 8, 16)
    dec = codes.view(torch.float8_e4m3fn).float() * sc.permute(0, 2, 1)[..., None]
    assert (dec - x).abs().max() <= x.abs().max() * 2 ** -3


def test_attention_byte_accounting():
    # 1 token, kv_len 10, KV=8, HD=128: 10*8*(256+8) + 2*16*128*2
    assert workloads.attention_bytes([10]) == 10 * 8 * 264 + 2 * 16 * 128 * 2
    assert workloads.attention_bytes([10], per_tensor=True) == 10 * 8 * 256 + 2 * 16 * 128 * 2
