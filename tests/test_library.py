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


@pytest.mark.skipif(torch.cuda.is_available(), reason="passes dummy device pointers; CPU-only check")
def test_gemm_argument_validation_without_device():
    lib = _lib.lib()
    ok, bad, unsup = _lib.CVH_OK, _lib.CVH_ERR_INVALID_ARG, _lib.CVH_ERR_UNSUPPORTED
    p = C.c_void_p(16)
    assert lib.cvh_gemm_bf16_nt(None, None, None, 0, 64, 256, 0, None) == ok           # M == 0: no-op
    assert lib.cvh_gemm_bf16_nt(None, p, p, 4, 64, 256, 0, None) == bad
    assert lib.cvh_gemm_bf16_nt(p, p, p, -1, 64, 256, 0, None) == bad
    assert lib.cvh_gemm_bf16_nt(p, p, p, 4, 56, 256, 0, None) == unsup                 # N % 16
    assert lib.cvh_gemm_bf16_nt(p, p, p, 4, 64, 200, 0, None) == unsup                 # K % 128
    assert lib.cvh_gemm_bf16_nt(p, p, p, 4, 64, 256, 77, None) == unsup                # unknown code
    assert lib.cvh_gemm_bf16_nt(p, p, p, 4, 64, 256, 10211, None) == unsup             # one-shot K fixed at 1024
    assert lib.cvh_gemm_bf16_nt(p, p, p, 4, 48, 256, 324222, None) == unsup            # 64-wide tile, N = 48
    assert lib.cvh_gemm_bf16_nt_swiglu(None, None, None, 0, 64, 256, 0, None) == ok
    assert lib.cvh_gemm_bf16_nt_swiglu(p, p, p, 4, 40, 256, 0, None) == unsup          # I % 16
    assert lib.cvh_gemm_bf16_nt_swiglu(p, p, p, 4, 64, 256, 11, None) == unsup         # not a SwiGLU code


def test_fused_gemm_and_prefill_plan_argument_validation_without_device():
    """The fused-epilogue projections and the prefill plan reject bad arguments, unsupported shapes
    and short workspaces before any device call; their automatic tiles are compiled ones."""
    lib = _lib.lib()
    ok, bad, unsup, wsp = _lib.CVH_OK, _lib.CVH_ERR_INVALID_ARG, _lib.CVH_ERR_UNSUPPORTED, _lib.CVH_ERR_WORKSPACE
    p = C.c_void_p(16)
    assert lib.cvh_gemm_bf16_nt_residual(None, None, None, None, 0, 1024, 2048, 0, None) == ok
    assert lib.cvh_gemm_bf16_nt_residual(p, None, p, p, 4, 1024, 2048, 0, None) == bad         # no row_ss
    assert lib.cvh_gemm_bf16_nt_residual(p, p, p, p, 4, 1000, 2048, 0, None) == unsup          # N % 16
    assert lib.cvh_gemm_bf16_nt_residual(p, p, p, p, 4, 1024, 2000, 0, None) == unsup          # K % 128
    assert lib.cvh_gemm_bf16_nt_residual(p, p, p, p, 4, 1024, 2048, 11, None) == unsup         # not a fused tile
    assert lib.cvh_gemm_bf16_nt_swiglu_rownorm(p, p, p, 1e-6, p, 4, 3072, 1152, 0, None) == unsup  # K % 256
    assert lib.cvh_gemm_bf16_nt_swiglu_rownorm(p, p, p, 1e-6, p, 4, 3072, 2048, 0, None) == unsup  # K > 1024
    assert lib.cvh_gemm_bf16_nt_swiglu_rownorm(p, p, None, 1e-6, p, 4, 3072, 1024, 0, None) == bad
    qkv = lambda *tail: lib.cvh_gemm_qkv_norm_rope_kv_write_fp8(p, p, None, 1e-6, *([p] * 11), *tail)  # noqa: E731
    assert qkv(0, 1024, 16, 8, 128, 16, 0, 1e-6, 0, None) == ok
    assert qkv(4, 1024, 16, 8, 64, 16, 0, 1e-6, 0, None) == unsup                             # head_dim 128 only
    assert qkv(4, 1024, 16, 8, 128, 24, 0, 1e-6, 0, None) == unsup                            # block size
    assert qkv(4, 1024, 16, 8, 128, 16, 5, 1e-6, 0, None) == unsup                            # scale mode
    assert qkv(-1, 1024, 16, 8, 128, 16, 0, 1e-6, 0, None) == bad
    fused = {k: set(_codes(lambda b, n, k=k: lib.cvh_gemm_fused_configs(k, b, n))) for k in range(3)}
    for M in (1, 15, 16, 64, 65, 128, 129, 256):
        for k in range(3):
            assert lib.cvh_gemm_fused_config(k, M) in fused[k], (k, M)
    assert all(c % 10 * ((c // 100) % 10) * 16 % 128 == 0 for c in fused[2])                 # whole heads
    # prefill plan: workspace of two int32 per 64-token group
    assert lib.cvh_paged_attention_prefill_workspace_bytes(0) == 0
    assert lib.cvh_paged_attention_prefill_workspace_bytes(65) == 2 * 2 * 4
    assert lib.cvh_paged_attention_prefill_plan(None, None, 0, 4, 16, None, 0, None) == ok
    assert lib.cvh_paged_attention_prefill_plan(p, p, 100, 4, 16, p, 15, None) == wsp
    assert lib.cvh_paged_attention_prefill_plan(p, p, 100, 4, 24, p, 16, None) == unsup
    assert lib.cvh_paged_attention_fp8_prefill_planned(*[p] * 7, 4, p, p, 100, 16, 8, 128, 16, 0, 0.1, p, 15,
                                                       None) == wsp


def _codes(fn):
    n = fn(None, 0)
    buf = (C.c_int * n)()
    assert fn(buf, n) == n
    return list(buf)


def test_gemm_dispatch_tables():
    """The automatic choice is a compiled configuration that fits the shape, for every projection
    of Qwen3-0.6B and every decode batch size, and the generic fallback covers other shapes."""
    lib = _lib.lib()
    every = set(_codes(lib.cvh_gemm_bf16_nt_configs))
    swiglu = set(_codes(lib.cvh_gemm_bf16_nt_swiglu_configs))
    assert len(every) == lib.cvh_gemm_bf16_nt_configs(None, 0) and swiglu

    def fits(code, N, K):
        if code >= 100000:
            return N % (16 * ((code // 100) % 10) * (code % 10)) == 0 and K % 128 == 0
        nwn = code % 10
        if code >= 10000:
            return N % (16 * nwn) == 0 and K == (4 // nwn) * ((code // 100) % 100) * 128
        return N % (16 * nwn) == 0 and K % ((4 // nwn) * 128) == 0

    shapes = [(4096, 1024), (1024, 2048), (6144, 1024), (1024, 3072), (151936, 1024), (512, 640), (96, 384)]
    for N, K in shapes:
        for M in (1, 2, 7, 8, 9, 16, 17, 33, 64, 65, 100, 128, 129, 200, 256, 1000, 4096):
            c = lib.cvh_gemm_bf16_nt_config(M, N, K)
            assert c in every and fits(c, N, K), (N, K, M, c)
    for M in (1, 16, 64, 65, 128, 129, 256):
        c = lib.cvh_gemm_bf16_nt_swiglu_config(M, 3072, 1024)
        assert c in swiglu and fits(c, 6144, 1024), (M, c)


def test_partition_policy_and_workspace_sizes():
    lib = _lib.lib()
    # headline decode (256 tokens, 8 kv heads = one 8-wave row group, 8 x 256-token blocks):
    # 256 partitions (2048 resident waves / 8)
    assert lib.cvh_paged_attention_partitions(256, 16, 8, 128, 8, 256) == 256
    rows, slots = 256, 256 * 2 * 16     # [G][2][WPG*REP] partial slots
    r256 = lambda v: (v + 255) // 256 * 256
    # plan: int2 token metadata [T] + int32 shared-prefix keys [T] + 184-byte workgroup records [G]
    # (first piece and tiles, row range, row window of 9 prefix entries and 8 token records)
    want = r256((rows + 1) * 4) + r256(slots * 128 * 4) + r256(slots * 2 * 4) + r256(256 * 8) + r256(256 * 4) + \
        r256(256 * 184)
    assert lib.cvh_paged_attention_workspace_bytes(256, 16, 8, 128, 8, 256, 0) == want
    # GQA 4 / 8 at head_dim 128 run on MFMA with one wave per physical kv head: the same 256 rows,
    # partial slots for all H query heads of a row group
    for H in (32, 64):
        want_m = r256(257 * 4) + r256(256 * 2 * H * 128 * 4) + r256(256 * 2 * H * 2 * 4) + r256(256 * 8) + \
            r256(256 * 4) + r256(256 * 184)
        assert lib.cvh_paged_attention_workspace_bytes(256, H, 8, 128, 8, 256, 0) == want_m, H
    # at head_dim 64 they run as 2 / 4 virtual kv heads of 2 query heads per kv head: twice / four
    # times the rows (prefix), the same partial slots per query head
    for H, vrows in ((32, 512), (64, 1024)):
        want_v = r256((vrows + 1) * 4) + r256(256 * 2 * H // (vrows // 256) * 64 * 4) + \
            r256(256 * 2 * H // (vrows // 256) * 2 * 4) + r256(256 * 8) + r256(256 * 4) + r256(256 * 184)
        assert lib.cvh_paged_attention_workspace_bytes(256, H, 8, 64, 8, 256, 0) == want_v, H
    # small batches: never less than two tiles per partition
    assert lib.cvh_paged_attention_partitions(1, 1, 1, 128, 1, 16) == 1
    # few rows: at most 8 partitions per row (8 rows -> 64, though 2 tiles each would allow 128)
    assert lib.cvh_paged_attention_partitions(8, 16, 8, 128, 4, 256) == 64
    assert lib.cvh_paged_attention_partitions(16, 16, 8, 128, 8, 256) == 128
    # one kv head: one-wave workgroups, capped at 1024 (not one per resident wave slot, 2048)
    assert lib.cvh_paged_attention_partitions(256, 2, 1, 128, 8, 256) == 1024
    assert lib.cvh_paged_attention_partitions(256, 4, 2, 128, 8, 256) == 1024
    # GQA 4 at head_dim 64: the policy sees the launch's virtual kv heads (16 = 2 row groups per
    # token), so 16 tokens give 32 rows and up to 8 partitions each: 256, as the launch and the
    # workspace size use; at head_dim 128 (MFMA, 16 rows): 128
    assert lib.cvh_paged_attention_partitions(16, 32, 8, 64, 8, 256) == 256
    r16 = r256(33 * 4) + r256(256 * 2 * 16 * 64 * 4) + r256(256 * 2 * 16 * 2 * 4) + r256(16 * 8) + \
        r256(16 * 4) + r256(256 * 184)
    assert lib.cvh_paged_attention_workspace_bytes(16, 32, 8, 64, 8, 256, 0) == r16
    assert lib.cvh_paged_attention_partitions(16, 32, 8, 128, 8, 256) == 128
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


def test_noalloc_array_holds_every_automatic_workspace():
    """cvh_paged_attention_fp8_noalloc accepts every launch with automatic partitions: the
    workspace of each supported head layout (GQA 1-8, head_dim 64/128, 1-64 kv heads), at every
    token count up to the 8192-row limit, fits the fixed array."""
    lib = _lib.lib()
    mx = lib.cvh_paged_attention_noalloc_max_workspace()
    worst = 0
    for hd in (64, 128):
        for kv in (1, 2, 3, 4, 8, 16, 32, 64):
            for rep in (1, 2, 4, 8):
                nkv = kv * (rep // 2 if (rep > 2 and hd != 128) else 1)   # the kernel's (virtual) kv heads
                wpg = 8 if nkv % 8 == 0 else 4 if nkv % 4 == 0 else 2 if nkv % 2 == 0 else 1
                tmax = 8192 // (nkv // wpg)                               # rows = T x row groups <= 8192
                for T in sorted({1, 7, 64, 256, 1000, max(1, tmax)}):
                    for W, bs in ((1, 16), (8, 256), (160, 256), (4096, 16)):
                        n = lib.cvh_paged_attention_workspace_bytes(T, kv * rep, kv, hd, W, bs, 0)
                        assert 0 < n <= mx, (hd, kv, rep, T, W, bs, n)
                        worst = max(worst, n)
    assert worst > mx // 2     # the bound is tight to within a factor of two (GQA 8: ~16.5 MiB)


@pytest.mark.skipif(torch.cuda.is_available(), reason="passes dummy device pointers; CPU-only check")
def test_runner_create_validates_before_allocating():
    """cvh_runner_create rejects bad descriptions before any device call: missing pointers,
    shapes the decode projections do not take, and fused-epilogue windows on shapes the fused
    projections do not take; handles it did not hand out are refused by every runner entry point."""
    lib = _lib.lib()
    L = 2
    layers = (_lib.RunnerLayer * L)()
    for i in range(L):
        for name, _ in _lib.RunnerLayer._fields_:
            setattr(layers[i], name, 4096)
    def desc(**kw):
        d = dict(n_layers=L, dim=1024, n_heads=16, n_kv_heads=8, head_dim=128, intermediate=3072, vocab=151936,
                 norm_eps=1e-6, attn_scale=0.088, block_size=256, scale_mode=0, max_batch=32, table_width=8,
                 scratch_block=100, fused_min_rows=16, fused_max_rows=256, embed=4096, final_norm=4096,
                 unit_gain=4096, rope_cos=4096, rope_sin=4096, hidden=4096, layers=layers)
        d.update(kw)
        return _lib.RunnerDesc(**d)
    h = C.c_void_p()
    bad, unsup = _lib.CVH_ERR_INVALID_ARG, _lib.CVH_ERR_UNSUPPORTED
    assert lib.cvh_runner_create(None, C.byref(h)) == bad
    assert lib.cvh_runner_create(C.byref(desc(embed=None)), C.byref(h)) == bad
    assert lib.cvh_runner_create(C.byref(desc(max_batch=257)), C.byref(h)) == bad
    assert lib.cvh_runner_create(C.byref(desc(n_heads=12)), C.byref(h)) == bad          # 12 % 8 != 0
    assert lib.cvh_runner_create(C.byref(desc(intermediate=3000)), C.byref(h)) == unsup  # K % 128 != 0
    assert lib.cvh_runner_create(C.byref(desc(dim=2048)), C.byref(h)) == unsup           # fused rows <= 1024
    layers[1].w_qkv_folded = None
    assert lib.cvh_runner_create(C.byref(desc()), C.byref(h)) == bad                      # fused weights missing
    assert h.value is None
    for fn, args in ((lib.cvh_runner_forward, (4, 0, None)), (lib.cvh_runner_capture, (4, 0)),
                     (lib.cvh_runner_replay, (4, 0, None)), (lib.cvh_runner_destroy, ())):
        assert fn(C.c_void_p(4096), *args) == bad
