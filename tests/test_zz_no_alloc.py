"""The no-allocation attention entry point (cvh_paged_attention_fp8_noalloc), through the C ABI.

It runs the kernels of cvh_paged_attention_fp8_ex with the split workspace in a fixed device array
of the library instead of a caller buffer, so its outputs must equal that call's bit for bit.
Two calls in a row, the second smaller, check that nothing left in the shared array by one call
leaks into the next; the oracle checks rows of the second call; a call whose workspace would not
fit the array is rejected before anything runs."""
import ctypes as C

import numpy as np
import pytest
import torch

from cppvllm_amd import _lib, workloads
from tests._util import assert_close_bf16, bits, np_, say

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _noalloc():
    lib = _lib.lib()
    return lib.cvh_paged_attention_fp8_noalloc, lib.cvh_paged_attention_noalloc_max_workspace


def _args(b, out):
    T, H, HD = b["q"].shape
    mode = _lib.SCALE_PER_TENSOR if b["k_scale"].numel() == 1 else _lib.SCALE_PER_TOKEN_HEAD
    return (out.data_ptr(), b["q"].data_ptr(), b["k_cache"].data_ptr(), b["v_cache"].data_ptr(),
            b["k_scale"].data_ptr(), b["v_scale"].data_ptr(), b["block_tables"].data_ptr(),
            b["block_tables"].shape[1], b["token_seq"].data_ptr(), b["token_kv_len"].data_ptr(), T, H,
            b["n_kv_heads"], HD, b["block_size"], mode, b["scale"])


def run_with_workspace(b, partitions=0):
    """The existing entry point, cvh_paged_attention_fp8_ex, with a caller-owned workspace."""
    lib = _lib.lib()
    T, H, HD = b["q"].shape
    W = b["block_tables"].shape[1]
    n = lib.cvh_paged_attention_workspace_bytes(T, H, b["n_kv_heads"], HD, W, b["block_size"], partitions)
    ws = torch.empty(n, dtype=torch.uint8, device=DEV)
    out = torch.full_like(b["q"], float("nan"))
    rc = lib.cvh_paged_attention_fp8_ex(*_args(b, out), partitions, ws.data_ptr(), n,
                                        torch.cuda.current_stream().cuda_stream)
    assert rc == 0, rc
    torch.cuda.synchronize()
    return bits(out)


def run_noalloc(b, partitions=0):
    fn, _ = _noalloc()
    out = torch.full_like(b["q"], float("nan"))
    rc = fn(*_args(b, out), partitions, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, rc
    torch.cuda.synchronize()
    return bits(out)


def test_noalloc_equals_workspace_call_twice(orc):
    say("no-alloc attention: config 3 (256 seqs) then 40 seqs, vs the workspace call")
    big = workloads.config3(device=DEV)
    small = workloads.config3(device=DEV, seqs=40, seed=1013)
    got_big = run_noalloc(big)
    assert np.array_equal(got_big, run_with_workspace(big))
    got_small = run_noalloc(small)
    assert np.array_equal(got_small, run_with_workspace(small))
    # an explicit partition count, then the automatic one again
    assert np.array_equal(run_noalloc(small, 300), run_with_workspace(small, 300))
    assert np.array_equal(run_noalloc(small), got_small)
    rows = list(range(0, 40, 3))
    cpu = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in small.items()}
    want = orc.paged_attention_fp8(np_(cpu["q"])[rows].copy(), np_(cpu["k_cache"]), np_(cpu["v_cache"]),
                                   np_(cpu["k_scale"]), np_(cpu["v_scale"]), np_(cpu["block_tables"]),
                                   np_(cpu["token_seq"])[rows].copy(), np_(cpu["token_kv_len"])[rows].copy(),
                                   cpu["n_heads"], cpu["n_kv_heads"], cpu["head_dim"], cpu["block_size"],
                                   orc.PER_TOKEN_HEAD, cpu["scale"])
    assert_close_bf16(got_small[rows], want)


@pytest.mark.parametrize("H", [32, 64])
def test_noalloc_gqa_mfma_twice(H):
    """GQA 4 / 8 (the MFMA decode path, the largest automatic workspaces) at config-3 size, then
    a smaller batch: bit for bit the workspace call."""
    say(f"no-alloc attention: GQA {H // 8} config 3 then 24 seqs")
    fn, mx = _noalloc()
    for seqs, seed in ((256, 1003), (24, 1017)):
        b = workloads.config3(device="cpu", seqs=seqs, seed=seed)
        g = torch.Generator().manual_seed(H + seqs)
        b["n_heads"] = H
        b["q"] = torch.randn((seqs, H, 128), generator=g).to(torch.bfloat16)
        b = {k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in b.items()}
        n = _lib.lib().cvh_paged_attention_workspace_bytes(seqs, H, 8, 128, b["block_tables"].shape[1], 256, 0)
        assert 0 < n <= mx()
        assert np.array_equal(run_noalloc(b), run_with_workspace(b))


def test_noalloc_rejects_oversize_and_bad_args():
    say("no-alloc attention: size limit and argument checks (nothing launched)")
    fn, mx = _noalloc()
    assert mx() == 24 << 20
    lib = _lib.lib()
    T, H, KV, HD, W, BS = 256, 16, 8, 128, 8, 256
    assert lib.cvh_paged_attention_workspace_bytes(T, H, KV, HD, W, BS, 0) <= mx()
    assert lib.cvh_paged_attention_workspace_bytes(T, H, KV, HD, W, BS, 4096) > mx()
    # rejected before any pointer is used: a dummy buffer stands in for every tensor
    dummy = torch.zeros(16, dtype=torch.uint8, device=DEV)
    p = dummy.data_ptr()
    stream = torch.cuda.current_stream().cuda_stream
    assert fn(p, p, p, p, p, p, p, W, p, p, T, H, KV, HD, BS, 0, 1.0, 4096, stream) == _lib.CVH_ERR_WORKSPACE
    assert fn(p, p, p, p, p, p, p, 0, p, p, T, H, KV, HD, BS, 0, 1.0, 0, stream) == _lib.CVH_ERR_INVALID_ARG
    assert fn(p, p, p, p, p, p, p, W, p, p, T, H, KV, HD, BS, 0, 1.0, -1, stream) == _lib.CVH_ERR_INVALID_ARG
    null = C.c_void_p(0)
    assert fn(null, null, null, null, null, null, null, W, null, null, 0, H, KV, HD, BS, 0, 1.0, 0, stream) == 0
    torch.cuda.synchronize()
