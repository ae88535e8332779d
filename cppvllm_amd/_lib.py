"""ctypes binding of the C ABI in ``include/cppvllm_hip.h`` (library ``libcppvllm_hip.so``).

The library is the product: there is no fallback. ``lib()`` raises if the shared object is
missing or does not export a declared symbol.
"""
from __future__ import annotations

import ctypes as C
import os
import re
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libcppvllm_hip.so"
HEADER = PKG.parent / "include" / "cppvllm_hip.h"
RUNNER_HEADER = PKG.parent / "include" / "cppvllm_runner.h"

CVH_OK = 0
CVH_ERR_INVALID_ARG = 1
CVH_ERR_UNSUPPORTED = 2
CVH_ERR_WORKSPACE = 3
CVH_ERR_LAUNCH = 4
ERROR_NAMES = {0: "CVH_OK", 1: "CVH_ERR_INVALID_ARG", 2: "CVH_ERR_UNSUPPORTED", 3: "CVH_ERR_WORKSPACE",
               4: "CVH_ERR_LAUNCH"}

SCALE_PER_TOKEN_HEAD = 0
SCALE_PER_TENSOR = 1
DTYPE_BF16, DTYPE_F16, DTYPE_F32 = 0, 1, 2

vp, i64, i32, f64, f32, sz = C.c_void_p, C.c_int64, C.c_int, C.c_double, C.c_float, C.c_size_t

# name -> (restype, argtypes), in the order of include/cppvllm_hip.h
SIGNATURES = {
    "cvh_paged_attention_fp8": (i32, [vp, vp, vp, vp, vp, vp, vp, i64, vp, vp, i64, i32, i32, i32, i32, i32, f64,
                                      vp, sz, vp]),
    "cvh_paged_attention_fp8_ex": (i32, [vp, vp, vp, vp, vp, vp, vp, i64, vp, vp, i64, i32, i32, i32, i32, i32, f64,
                                         i32, vp, sz, vp]),
    "cvh_paged_attention_fp8_split_phase": (i32, [vp, vp, vp, vp, vp, vp, vp, i64, vp, vp, i64, i32, i32, i32, i32,
                                                  i32, f64, i32, vp, sz, vp]),
    "cvh_paged_attention_fp8_merge_phase": (i32, [vp, vp, vp, vp, vp, vp, vp, i64, vp, vp, i64, i32, i32, i32, i32,
                                                  i32, f64, i32, vp, sz, vp]),
    "cvh_paged_attention_fp8_prefill": (i32, [vp, vp, vp, vp, vp, vp, vp, i64, vp, vp, i64, i32, i32, i32, i32, i32,
                                              f64, vp]),
    "cvh_paged_attention_prefill_workspace_bytes": (sz, [i64]),
    "cvh_paged_attention_prefill_plan": (i32, [vp, vp, i64, i64, i32, vp, sz, vp]),
    "cvh_paged_attention_fp8_prefill_planned": (i32, [vp, vp, vp, vp, vp, vp, vp, i64, vp, vp, i64, i32, i32, i32, i32,
                                                      i32, f64, vp, sz, vp]),
    "cvh_paged_attention_plan": (i32, [vp, i64, vp, vp, i64, i32, i32, i32, i32, i32, vp, sz, vp]),
    "cvh_paged_attention_plan_shared": (i32, [vp, i64, vp, vp, vp, i64, i32, i32, i32, i32, i32, vp, sz, vp]),
    "cvh_paged_attention_fp8_planned_shared": (i32, [vp, vp, vp, vp, vp, vp, vp, i64, vp, vp, i64, i32, i32, i32, i32,
                                                     i32, f64, i32, vp, sz, vp]),
    "cvh_paged_attention_fp8_planned_shared_split_phase": (i32, [vp, vp, vp, vp, vp, vp, vp, i64, vp, vp, i64, i32, i32,
                                                                 i32, i32, i32, f64, i32, vp, sz, vp]),
    "cvh_paged_attention_fp8_planned_shared_merge_phase": (i32, [vp, vp, vp, vp, vp, vp, vp, i64, vp, vp, i64, i32, i32,
                                                                 i32, i32, i32, f64, i32, vp, sz, vp]),
    "cvh_paged_attention_fp8_planned": (i32, [vp, vp, vp, vp, vp, vp, vp, i64, vp, vp, i64, i32, i32, i32, i32, i32,
                                              f64, i32, vp, sz, vp]),
    "cvh_paged_attention_fp8_planned_split_phase": (i32, [vp, vp, vp, vp, vp, vp, vp, i64, vp, vp, i64, i32, i32, i32,
                                                          i32, i32, f64, i32, vp, sz, vp]),
    "cvh_paged_attention_fp8_noalloc": (i32, [vp, vp, vp, vp, vp, vp, vp, i64, vp, vp, i64, i32, i32, i32, i32, i32,
                                              f64, i32, vp]),
    "cvh_paged_attention_noalloc_max_workspace": (sz, []),
    "cvh_paged_attention_workspace_bytes": (sz, [i64, i32, i32, i32, i64, i32, i32]),
    "cvh_paged_attention_workspace_bytes_shared": (sz, [i64, i32, i32, i32, i64, i32, i32]),
    "cvh_paged_attention_partitions": (i32, [i64, i32, i32, i32, i64, i32]),
    "cvh_rms_norm": (i32, [vp, vp, vp, i64, i32, f64, i32, vp]),
    "cvh_add_rms_norm": (i32, [vp, vp, vp, vp, i64, i32, f64, i32, vp]),
    "cvh_qk_norm_rope_kv_write_fp8": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i32, i32,
                                            i32, i32, i32, f64, vp]),
    "cvh_build_token_metadata": (i32, [vp, i64, vp, i64, vp, i64, i32, vp, vp, vp, vp]),
    "cvh_rope_tables_host": (i32, [vp, vp, i64, i32, f64]),
    "cvh_fp8_e4m3_quantize": (i32, [vp, vp, i64, f32, vp]),
    "cvh_swiglu": (i32, [vp, vp, i64, i32, i32, vp]),
    "cvh_sample_tokens": (i32, [vp, vp, i32, vp, vp, i64, i32, C.c_uint64, C.c_uint64, vp]),
    "cvh_feed_tokens": (i32, [vp, vp, vp, i64, vp]),
    "cvh_embedding": (i32, [vp, vp, vp, i64, i32, i64, vp]),
    "cvh_gemm_bf16_nt": (i32, [vp, vp, vp, i64, i32, i32, i32, vp]),
    "cvh_gemm_bf16_nt_config": (i32, [i64, i32, i32]),
    "cvh_gemm_bf16_nt_configs": (i32, [vp, i32]),
    "cvh_gemm_bf16_nt_swiglu": (i32, [vp, vp, vp, i64, i32, i32, i32, vp]),
    "cvh_gemm_bf16_nt_swiglu_config": (i32, [i64, i32, i32]),
    "cvh_gemm_bf16_nt_swiglu_configs": (i32, [vp, i32]),
    "cvh_gemm_bf16_nt_residual": (i32, [vp, vp, vp, vp, i64, i32, i32, i32, vp]),
    "cvh_gemm_bf16_nt_swiglu_rownorm": (i32, [vp, vp, vp, f64, vp, i64, i32, i32, i32, vp]),
    "cvh_gemm_qkv_norm_rope_kv_write_fp8": (i32, [vp, vp, vp, f64, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i64,
                                                  i32, i32, i32, i32, i32, i32, f64, i32, vp]),
    "cvh_gemm_fused_configs": (i32, [i32, vp, i32]),
    "cvh_gemm_fused_config": (i32, [i32, i64]),
    "cvh_version": (C.c_char_p, []),
    # include/cppvllm_runner.h
    "cvh_runner_create": (i32, [vp, vp]),
    "cvh_runner_destroy": (i32, [vp]),
    "cvh_runner_stage": (i32, [vp, i32, i64, i32, vp, vp, vp, i64, vp, vp, vp, vp]),
    "cvh_runner_forward": (i32, [vp, i32, i32, vp]),
    "cvh_runner_capture": (i32, [vp, i32, i32]),
    "cvh_runner_replay": (i32, [vp, i32, i32, vp]),
}


class RunnerLayer(C.Structure):
    """struct cvh_runner_layer (include/cppvllm_runner.h)."""
    _fields_ = [(n, vp) for n in ("w_qkv", "w_qkv_folded", "w_o", "w_gate_up", "w_gate_up_folded", "w_down",
                                  "attn_norm", "ffn_norm", "q_norm", "k_norm", "k_cache", "v_cache", "k_scale",
                                  "v_scale")]


class RunnerDesc(C.Structure):
    """struct cvh_runner_desc (include/cppvllm_runner.h)."""
    _fields_ = [("n_layers", i32), ("dim", i32), ("n_heads", i32), ("n_kv_heads", i32), ("head_dim", i32),
                ("intermediate", i32), ("vocab", i64), ("norm_eps", f64), ("attn_scale", f64), ("block_size", i32),
                ("scale_mode", i32), ("max_batch", i32), ("table_width", i64), ("scratch_block", i64),
                ("fused_min_rows", i32), ("fused_max_rows", i32), ("embed", vp), ("final_norm", vp),
                ("unit_gain", vp), ("rope_cos", vp), ("rope_sin", vp), ("hidden", vp),
                ("layers", C.POINTER(RunnerLayer))]

_LIB = None


class CvhError(RuntimeError):
    """A non-zero status returned across the C ABI."""

    def __init__(self, fn: str, code: int):
        super().__init__(f"{fn} failed: {ERROR_NAMES.get(code, code)}")
        self.code = code


def header_symbols() -> list[str]:
    """Function names declared in include/cppvllm_hip.h."""
    text = HEADER.read_text() + RUNNER_HEADER.read_text()
    return sorted(set(re.findall(r"\b(cvh_[a-z0-9_]+)\s*\(", text)))


def lib() -> C.CDLL:
    """Load libcppvllm_hip.so (built by cppvllm_amd.build). Raises if it is missing."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = Path(os.environ.get("CVH_LIB", LIB_PATH))
    if not path.exists():
        raise RuntimeError(f"{path} is missing: build it with `python -m cppvllm_amd.build` "
                           "(the HIP library is required; there is no fallback path)")
    handle = C.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = handle
    return handle


def check(fn: str, code: int) -> None:
    if code != CVH_OK:
        raise CvhError(fn, code)
