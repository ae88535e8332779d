"""CPU fuzz of the C ABI: every device entry point called with edge-value integers (negative,
zero, one, powers of two, values past every documented limit), null or dummy device pointers and
the default stream. Without a GPU nothing can run, so each call must come back with one of the
defined status codes: rejected by validation, or CVH_ERR_LAUNCH from the runtime, never a crash
or an undefined code. Host-side helpers that write through their pointer arguments are left out."""
import ctypes as C
import random

import pytest
import torch

from cppvllm_amd import _lib

# host functions that write to host memory through their pointers, and argument-free queries
SKIP = {"cvh_rope_tables_host", "cvh_gemm_bf16_nt_configs", "cvh_gemm_bf16_nt_swiglu_configs",
        "cvh_gemm_fused_configs", "cvh_version",
        # the runner's create / stage read and write host structs and arrays through their pointers
        "cvh_runner_create", "cvh_runner_stage"}
I64 = [-(1 << 40), -1, 0, 1, 2, 3, 16, 63, 64, 65, 255, 4097, 8192, 8193, 1 << 20, 1 << 31, 1 << 40]
I32 = [-7, -1, 0, 1, 2, 3, 4, 8, 16, 24, 64, 96, 128, 256, 1000, 1024, 4096, 8192, 1 << 30, (1 << 31) - 1]
# pure queries: they return a size, a count or a configuration code, not a status
QUERIES = {"cvh_gemm_bf16_nt_config", "cvh_gemm_bf16_nt_swiglu_config", "cvh_gemm_fused_config",
           "cvh_paged_attention_partitions", "cvh_paged_attention_workspace_bytes",
           "cvh_paged_attention_workspace_bytes_shared",
           "cvh_paged_attention_prefill_workspace_bytes", "cvh_paged_attention_noalloc_max_workspace"}
F64 = [0.0, 1e-6, 0.088, 1.0, -1.0, float("inf"), float("nan")]
SZ = [0, 16, 1 << 20, 1 << 40]


def _arg(t, rng, last):
    if t is C.c_void_p:
        return None if last else rng.choice([None, C.c_void_p(4096)])
    if t is C.c_int64:
        return rng.choice(I64)
    if t is C.c_int32:
        return rng.choice(I32)
    if t is C.c_double:
        return rng.choice(F64)
    if t is C.c_size_t:
        return rng.choice(SZ)
    if t is C.c_float:
        return rng.choice(F64)
    raise TypeError(t)


@pytest.mark.skipif(torch.cuda.is_available(), reason="dummy device pointers must not reach a real GPU")
@pytest.mark.parametrize("name", sorted(set(_lib.SIGNATURES) - SKIP))
def test_entry_point_returns_a_status_for_any_arguments(name):
    lib = _lib.lib()
    fn = getattr(lib, name)
    ret, argt = _lib.SIGNATURES[name]
    rng = random.Random(hash(name) & 0xFFFF)
    for _ in range(300):
        args = [_arg(t, rng, i == len(argt) - 1) for i, t in enumerate(argt)]
        r = fn(*args)
        if name in QUERIES:
            assert r >= 0, (name, args, r)
        else:
            assert r in _lib.ERROR_NAMES, (name, args, r)
