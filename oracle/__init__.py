"""CPU oracle for the FP8 paged-decode hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package. It is the checker, never the thing measured or shipped: the product
(``cppvllm_amd``) never imports it.

The restatement lives in ``cvh_oracle.c`` (built by ``oracle/Makefile`` into ``liborc.so``);
this module wraps it for numpy arrays. bf16 values travel as ``np.uint16`` bit patterns.

How each function is pinned (independently of the code it checks; tests/test_oracle.py):
  * e4m3_encode   — torch.float8_e4m3fn cast (after clamping to +-448) over every float32
                    bit pattern class: all 2^16 upper-half patterns x low-bit variants, every
                    e4m3 midpoint and boundary; saturation/NaN special cases by closed form.
  * e4m3_decode   — all 256 codes vs the OCP spec formula evaluated in numpy and vs torch.
  * bf16 / f16    — torch's float32->bfloat16 / ->float16 casts over random + edge patterns.
  * rms_norm, add_rms_norm — numpy float64 recomputation (agrees to 1 ulp of the output
                    dtype), closed-form constant rows (x = c => inv = 1/sqrt(c^2+eps)).
  * qk_norm_rope_kv_write_fp8 — numpy float64 recomputation of norm + RoPE (Q within 1 bf16
                    ulp), pos = 0 => RoPE identity, zero heads => scale 1e-8/448 and zero bytes,
                    V bytes/scales by the order-free closed form (bit-exact), slot indexing by
                    brute-force inverse mapping, slot = -1 rows untouched.
  * paged_attention_fp8 — float64 brute-force softmax over decoded K/V (numpy), known answers
                    (kv_len = 1 => out = decoded v0; identical keys => mean of V; dominant key),
                    permutation invariance of physical block ids.
  * token_metadata — numpy searchsorted(right=True) + gather closed form.
  * rope tables   — numpy float64 cos/sin of pos * theta^(-2i/hd).
  * swiglu        — numpy float64 silu then the two roundings via torch casts; g = 0 => 0,
                    large |g| limits (silu(g) -> g, -> -0).
  * philox4x32_10 — the Random123 known-answer vectors for philox4x32_10.
  * sample_tokens — numpy argmax (first maximum) for greedy rows; Gumbel rows: the u stream's
                    closed form from the KAT-pinned Philox and a numpy float64 score + argmax.
There are no golden vectors in the reference (it has no tests); no function is left unpinned.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liborc.so"
PER_TOKEN_HEAD, PER_TENSOR = 0, 1
BF16, F16, F32 = 0, 1, 2

_L = None


def build() -> Path:
    subprocess.run(["make", "-s", "-B", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _L
    if _L is None:
        if not LIB_PATH.exists():
            build()
        _L = C.CDLL(str(LIB_PATH))
        vp, i64, i32, f64, f32 = C.c_void_p, C.c_int64, C.c_int, C.c_double, C.c_float
        sig = {
            "orc_f32_to_bf16": (C.c_uint16, [f32]),
            "orc_e4m3_encode": (C.c_uint8, [f32]),
            "orc_e4m3_decode": (f32, [C.c_uint8]),
            "orc_e4m3_quantize": (None, [vp, vp, i64, f32]),
            "orc_rms_norm": (None, [vp, vp, vp, i64, i32, f64, i32]),
            "orc_add_rms_norm": (None, [vp, vp, vp, vp, i64, i32, f64, i32]),
            "orc_qk_norm_rope_kv_write_fp8": (None, [vp] * 14 + [i64, i32, i32, i32, i32, i32, f64]),
            "orc_paged_attention_fp8": (None, [vp] * 7 + [i64, vp, vp, i64, i32, i32, i32, i32, i32, f64]),
            "orc_token_metadata": (None, [vp, i64, vp, i64, vp, i64, i32, vp, vp, vp]),
            "orc_swiglu": (None, [vp, vp, i64, i32, i32]),
            "orc_philox4x32_10": (None, [vp, C.c_uint32, C.c_uint32]),
            "orc_sample_tokens": (None, [vp, vp, i32, vp, vp, i64, i32, C.c_uint64, C.c_uint64]),
            "orc_max_threads": (i32, []),
            "orc_set_threads": (None, [i32]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(_L, name)
            fn.restype = res
            fn.argtypes = args
    return _L


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def max_threads() -> int:
    return int(lib().orc_max_threads())


# ---- element conversions --------------------------------------------------------------------------
def e4m3_quantize(x: np.ndarray, inv_scale: float = 1.0) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint8)
    lib().orc_e4m3_quantize(_p(out), _p(x), x.size, float(inv_scale))
    return out


def e4m3_decode_table() -> np.ndarray:
    return np.array([lib().orc_e4m3_decode(c) for c in range(256)], dtype=np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (RNE) using the oracle's own rounding."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    f = lib().orc_f32_to_bf16
    return np.array([f(float(v)) for v in x], dtype=np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---- norms -------------------------------------------------------------------------------------------
def rms_norm(x: np.ndarray, w: np.ndarray, eps: float, dtype: int = BF16) -> np.ndarray:
    x = np.ascontiguousarray(x)
    w = np.ascontiguousarray(w)
    out = np.empty_like(x)
    lib().orc_rms_norm(_p(out), _p(x), _p(w), x.shape[0], x.shape[1], float(eps), dtype)
    return out


def add_rms_norm(resid: np.ndarray, x: np.ndarray, w: np.ndarray, eps: float, dtype: int = BF16):
    """Returns (new_resid, out); the inputs are not modified."""
    r = np.array(resid, copy=True, order="C")
    x = np.ascontiguousarray(x)
    w = np.ascontiguousarray(w)
    out = np.empty_like(x)
    lib().orc_add_rms_norm(_p(r), _p(x), _p(w), _p(out), r.shape[0], r.shape[1], float(eps), dtype)
    return r, out


# ---- qk-norm / rope / fp8 kv write ---------------------------------------------------------------------
def qk_norm_rope_kv_write_fp8(qkv, q_norm, k_norm, cos, sin, positions, slots, k_cache, v_cache, k_scale, v_scale,
                              n_heads, n_kv_heads, head_dim, block_size, scale_mode=PER_TOKEN_HEAD, eps=1e-6,
                              dense=False):
    """Writes k_cache/v_cache/(k_scale/v_scale) in place. Returns (q_out, k_dense, v_dense)."""
    T = positions.shape[0]
    q_out = np.zeros((T, n_heads, head_dim), dtype=np.uint16)
    kd = np.zeros((T, n_kv_heads, head_dim), dtype=np.uint16) if dense else None
    vd = np.zeros((T, n_kv_heads, head_dim), dtype=np.uint16) if dense else None
    lib().orc_qk_norm_rope_kv_write_fp8(
        _p(q_out), _p(qkv), _p(q_norm), _p(k_norm), _p(cos), _p(sin), _p(positions), _p(slots), _p(k_cache),
        _p(v_cache), _p(k_scale), _p(v_scale), _p(kd), _p(vd), T, n_heads, n_kv_heads, head_dim, block_size,
        scale_mode, float(eps))
    return q_out, kd, vd


# ---- paged attention -------------------------------------------------------------------------------------
def paged_attention_fp8(q, k_cache, v_cache, k_scale, v_scale, block_tables, token_seq, token_kv_len, n_heads,
                        n_kv_heads, head_dim, block_size, scale_mode=PER_TOKEN_HEAD, scale=None) -> np.ndarray:
    T = token_kv_len.shape[0]
    if scale is None:
        scale = 1.0 / np.sqrt(head_dim)
    out = np.zeros((T, n_heads, head_dim), dtype=np.uint16)
    lib().orc_paged_attention_fp8(_p(out), _p(q), _p(k_cache), _p(v_cache), _p(k_scale), _p(v_scale),
                                  _p(block_tables), block_tables.shape[1], _p(token_seq), _p(token_kv_len), T,
                                  n_heads, n_kv_heads, head_dim, block_size, scale_mode, float(scale))
    return out


def token_metadata(cu_seqlens, positions, block_tables, block_size):
    T = positions.shape[0]
    S = cu_seqlens.shape[0] - 1
    seq = np.empty(T, dtype=np.int64)
    slot = np.empty(T, dtype=np.int64)
    kvl = np.empty(T, dtype=np.int64)
    lib().orc_token_metadata(_p(cu_seqlens), S, _p(positions), T, _p(block_tables), block_tables.shape[1],
                             block_size, _p(seq), _p(slot), _p(kvl))
    return seq, slot, kvl


# ---- model ops around the path ------------------------------------------------------------------------
def swiglu(gate_up: np.ndarray, dtype: int = BF16) -> np.ndarray:
    """gate_up [N, 2I] (bf16/f16 bit patterns as uint16, or float32) -> out [N, I]."""
    gu = np.ascontiguousarray(gate_up)
    N, I2 = gu.shape
    out = np.empty((N, I2 // 2), dtype=gu.dtype)
    lib().orc_swiglu(_p(out), _p(gu), N, I2 // 2, dtype)
    return out


def philox4x32_10(counter, key) -> np.ndarray:
    c = np.array(counter, dtype=np.uint32)
    lib().orc_philox4x32_10(_p(c), int(key[0]), int(key[1]))
    return c


def sample_tokens(logits: np.ndarray, rows=None, temps=None, seed: int = 0, offset: int = 0) -> np.ndarray:
    """logits float32 or bf16 bit patterns (uint16) [*, V]; rows int64 [R] (None: all rows);
    temps float32 [R] (None: greedy)."""
    lg = np.ascontiguousarray(logits)
    dt = F32 if lg.dtype == np.float32 else BF16
    R = lg.shape[0] if rows is None else len(rows)
    rows = None if rows is None else np.ascontiguousarray(rows, dtype=np.int64)
    temps = None if temps is None else np.ascontiguousarray(temps, dtype=np.float32)
    out = np.empty(R, dtype=np.int64)
    lib().orc_sample_tokens(_p(out), _p(lg), dt, _p(rows), _p(temps), R, lg.shape[1], seed, offset)
    return out


if os.environ.get("CVH_ORACLE_REBUILD"):
    build()
