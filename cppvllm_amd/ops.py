"""Torch-tensor mirror of cppvllm's kernel-layer API, backed by the gfx950 C ABI.

Names, argument order and meaning follow the reference's free functions:
  * ``paged_attention_fp8``            — kernels/paged_attention.h:5-7
  * ``fused.rms_norm`` / ``add_rms_norm`` / ``qk_norm_rope_kv_write_fp8`` — kernels/fused_ops.h:7-15
Shapes that the reference reads from tensor metadata are read the same way here
(``q.size(1)`` = heads, ``k_cache.size(1)`` = block size, ``k_cache.size(2)`` = kv heads,
``block_tables.size(1)`` = table width; kernels/paged_attention.cu:398-400,432,463-464).
Errors the reference raises with TORCH_CHECK raise ``CvhError``/``ValueError`` here.

Every call goes to the HIP library on torch's current stream. There is no CPU or PyTorch fallback.
"""
from __future__ import annotations

import types

import torch

from . import _lib
from ._lib import SCALE_PER_TENSOR, SCALE_PER_TOKEN_HEAD, check

_DT = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16, torch.float32: _lib.DTYPE_F32}


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t):
    return None if t is None or (isinstance(t, torch.Tensor) and t.numel() == 0) else t.data_ptr()


def _require_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("cppvllm_amd ops take device tensors only")
        if t is not None and not t.is_contiguous():
            raise ValueError("cppvllm_amd ops take contiguous tensors only")


def _scale_mode(k_scale: torch.Tensor) -> int:
    return SCALE_PER_TENSOR if k_scale.numel() == 1 else SCALE_PER_TOKEN_HEAD


def paged_attention_workspace(num_tokens: int, n_heads: int, n_kv_heads: int, head_dim: int, table_width: int,
                              block_size: int, partitions: int = 0, device="cuda", shared: bool = False) -> torch.Tensor:
    """Preallocated split-K workspace (what the reference allocates per call, paged_attention.cu:415-421).
    shared=True: the layout of the prefix-sharing plan and launches (paged_attention_plan with
    shared_blocks, paged_attention_fp8(..., shared=True))."""
    L = _lib.lib()
    fn = L.cvh_paged_attention_workspace_bytes_shared if shared else L.cvh_paged_attention_workspace_bytes
    n = fn(num_tokens, n_heads, n_kv_heads, head_dim, table_width, block_size, partitions)
    return torch.empty(max(int(n), 1), dtype=torch.uint8, device=device)


def paged_attention_plan(block_tables, token_seq, token_kv_len, n_heads: int, n_kv_heads: int, head_dim: int,
                         block_size: int, workspace: torch.Tensor, partitions: int = 0,
                         shared_blocks: torch.Tensor | None = None) -> None:
    """Build the per-step plan that ``paged_attention_fp8(..., planned=True)`` reads from `workspace`
    (once per batch layout, before the layers of a step). shared_blocks (int32, one per table row):
    leading blocks each row shares with other rows (prefix-cache hits): tokens whose rows share them
    are grouped, and the shared launches read each group's shared K/V once per unit of up to
    16 / (query heads per kv head) tokens at head_dim 128 (needs a workspace made with shared=True)."""
    T = token_seq.size(0)
    if T == 0:
        return
    _require_cuda(block_tables, token_seq, token_kv_len, workspace, shared_blocks)
    L = _lib.lib()
    common = (T, int(n_heads), int(n_kv_heads), int(head_dim), int(block_size), int(partitions), workspace.data_ptr(),
              workspace.numel() * workspace.element_size(), _stream(token_seq))
    if shared_blocks is None:
        code = L.cvh_paged_attention_plan(block_tables.data_ptr(), block_tables.size(1), token_seq.data_ptr(),
                                          token_kv_len.data_ptr(), *common)
    else:
        if shared_blocks.dtype != torch.int32:
            raise ValueError("shared_blocks must be int32")
        code = L.cvh_paged_attention_plan_shared(block_tables.data_ptr(), block_tables.size(1), token_seq.data_ptr(),
                                                 token_kv_len.data_ptr(), shared_blocks.data_ptr(), *common)
    check("paged_attention_plan", code)


def paged_attention_fp8(out, q, k_cache, v_cache, k_scale, v_scale, block_tables, token_seq, token_kv_len,
                        scale: float, *, workspace: torch.Tensor | None = None, partitions: int = 0,
                        planned: bool = False, shared: bool = False) -> None:
    """FP8 paged attention over a ragged batch of query tokens (kernels/paged_attention.cu:459-473).

    out, q: bf16 [T, H, HD]; k_cache, v_cache: uint8 [NB, BS, KV, HD]; k_scale, v_scale: float32
    [NB, BS, KV] (memory order [NB][KV][BS]) or one element each (per-tensor); block_tables int64
    [S, W]; token_seq, token_kv_len int64 [T]. planned=True reads the plan that
    ``paged_attention_plan`` left in `workspace` for the same layout; shared=True runs the
    shared-prefix units of a plan built with shared_blocks.
    """
    T = q.size(0)
    if T == 0:
        return
    _require_cuda(out, q, k_cache, v_cache, k_scale, v_scale, block_tables, token_seq, token_kv_len)
    H, HD = q.size(1), q.size(2)
    BS, KV = k_cache.size(1), k_cache.size(2)
    W = block_tables.size(1)
    if workspace is None:
        if planned:
            raise ValueError("planned=True needs the workspace the plan was built in")
        workspace = paged_attention_workspace(T, H, KV, HD, W, BS, partitions, q.device)
    L = _lib.lib()
    fn = (L.cvh_paged_attention_fp8_planned_shared if shared else L.cvh_paged_attention_fp8_planned) if planned \
        else L.cvh_paged_attention_fp8_ex
    code = fn(
        out.data_ptr(), q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), k_scale.data_ptr(),
        v_scale.data_ptr(), block_tables.data_ptr(), W, token_seq.data_ptr(), token_kv_len.data_ptr(), T, H, KV,
        HD, BS, _scale_mode(k_scale), float(scale), int(partitions), workspace.data_ptr(),
        workspace.numel() * workspace.element_size(), _stream(q))
    check("paged_attention_fp8", code)


def prefill_supported(n_heads: int, n_kv_heads: int, head_dim: int) -> bool:
    """Shapes the MFMA multi-query kernel covers (else use paged_attention_fp8)."""
    return head_dim == 128 and n_heads % n_kv_heads == 0 and n_heads // n_kv_heads in (1, 2)


def prefill_workspace(num_tokens: int, device="cuda") -> torch.Tensor:
    """Workspace of paged_attention_prefill_plan for num_tokens query tokens."""
    n = int(_lib.lib().cvh_paged_attention_prefill_workspace_bytes(int(num_tokens)))
    return torch.empty((max(1, (n + 3) // 4),), dtype=torch.int32, device=device)


def paged_attention_prefill_plan(token_seq, token_kv_len, table_width: int, block_size: int, workspace) -> None:
    """Order the 64-token groups of a multi-query batch longest key walk first (once per step)."""
    T = token_seq.numel()
    if T == 0:
        return
    _require_cuda(token_seq, token_kv_len, workspace)
    check("paged_attention_prefill_plan", _lib.lib().cvh_paged_attention_prefill_plan(
        token_seq.data_ptr(), token_kv_len.data_ptr(), T, int(table_width), int(block_size), workspace.data_ptr(),
        workspace.numel() * workspace.element_size(), _stream(token_seq)))


def paged_attention_fp8_prefill(out, q, k_cache, v_cache, k_scale, v_scale, block_tables, token_seq, token_kv_len,
                                scale: float, *, workspace=None) -> None:
    """paged_attention_fp8 for multi-token query rows (chunked prefill) on the MFMA kernel: same
    arguments and result. workspace: a plan from paged_attention_prefill_plan over the same
    token_seq / token_kv_len (longest groups first, key tiles split over two half-workgroups)."""
    T = q.size(0)
    if T == 0:
        return
    _require_cuda(out, q, k_cache, v_cache, k_scale, v_scale, block_tables, token_seq, token_kv_len, workspace)
    H, HD = q.size(1), q.size(2)
    BS, KV = k_cache.size(1), k_cache.size(2)
    args = (out.data_ptr(), q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), k_scale.data_ptr(),
            v_scale.data_ptr(), block_tables.data_ptr(), block_tables.size(1), token_seq.data_ptr(),
            token_kv_len.data_ptr(), T, H, KV, HD, BS, _scale_mode(k_scale), float(scale))
    L = _lib.lib()
    if workspace is None:
        code = L.cvh_paged_attention_fp8_prefill(*args, _stream(q))
    else:
        code = L.cvh_paged_attention_fp8_prefill_planned(*args, workspace.data_ptr(),
                                                         workspace.numel() * workspace.element_size(), _stream(q))
    check("paged_attention_fp8_prefill", code)


def _rms_norm(out, x, w, eps):
    if x.size(0) == 0:
        return
    _require_cuda(out, x, w)
    code = _lib.lib().cvh_rms_norm(out.data_ptr(), x.data_ptr(), w.data_ptr(), x.size(0), x.size(1), float(eps),
                                   _DT[x.dtype], _stream(x))
    check("rms_norm", code)


def _add_rms_norm(resid, x, w, out, eps):
    if resid.size(0) == 0:
        return
    _require_cuda(resid, x, w, out)
    code = _lib.lib().cvh_add_rms_norm(resid.data_ptr(), x.data_ptr(), w.data_ptr(), out.data_ptr(), resid.size(0),
                                       resid.size(1), float(eps), _DT[resid.dtype], _stream(resid))
    check("add_rms_norm", code)


def _qk_norm_rope_kv_write_fp8(q_out, qkv, q_norm, k_norm, cos, sin, positions, slots, k_cache, v_cache, k_scale,
                               v_scale, k_dense, v_dense, n_heads: int, n_kv_heads: int, eps: float) -> None:
    T, HD = q_out.size(0), q_out.size(2)
    if T == 0:
        return
    _require_cuda(q_out, qkv, q_norm, k_norm, cos, sin, positions, slots, k_cache, v_cache, k_scale, v_scale)
    BS = k_cache.size(1)
    code = _lib.lib().cvh_qk_norm_rope_kv_write_fp8(
        q_out.data_ptr(), qkv.data_ptr(), q_norm.data_ptr(), k_norm.data_ptr(), cos.data_ptr(), sin.data_ptr(),
        positions.data_ptr(), slots.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), k_scale.data_ptr(),
        v_scale.data_ptr(), _ptr(k_dense), _ptr(v_dense), T, int(n_heads), int(n_kv_heads), HD, BS,
        _scale_mode(k_scale), float(eps), _stream(q_out))
    check("qk_norm_rope_kv_write_fp8", code)


def _swiglu(out, gate_up) -> None:
    """out [T, I] = silu(gate) * up over gate_up [T, 2I] (kernels/fused_ops.cu:261-283)."""
    if out.numel() == 0:
        return
    _require_cuda(out, gate_up)
    if gate_up.dtype != out.dtype or gate_up.size(-1) != 2 * out.size(-1):
        raise ValueError("swiglu: gate_up must be [T, 2I] of out's dtype")
    check("swiglu", _lib.lib().cvh_swiglu(out.data_ptr(), gate_up.data_ptr(), out.size(0), out.size(1),
                                          _DT[out.dtype], _stream(out)))


def _sample_tokens(out, logits, rows, temps, seed: int, offset: int) -> None:
    """out int64 [R] = sampled token of logits row rows[r] (kernels/fused_ops.cu:367-378); rows or
    temps may be None (all rows / greedy)."""
    R = out.numel() if rows is None else rows.numel()
    if R == 0:
        return
    _require_cuda(out, logits, rows, temps)
    ldt = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16}[logits.dtype]
    check("sample_tokens", _lib.lib().cvh_sample_tokens(out.data_ptr(), logits.data_ptr(), ldt, _ptr(rows),
                                                        _ptr(temps), R, logits.size(1), int(seed) & (2**64 - 1),
                                                        int(offset) & (2**64 - 1), _stream(logits)))


def _feed_tokens(tokens, src, prev) -> None:
    """tokens[i] = prev[src[i]] where src[i] >= 0 (kernels/fused_ops.cu:388-397)."""
    if tokens.numel() == 0:
        return
    _require_cuda(tokens, src, prev)
    check("feed_tokens", _lib.lib().cvh_feed_tokens(tokens.data_ptr(), src.data_ptr(), prev.data_ptr(),
                                                    tokens.numel(), _stream(tokens)))


# The reference's `namespace fused` (kernels/fused_ops.h:5).
fused = types.SimpleNamespace(rms_norm=_rms_norm, add_rms_norm=_add_rms_norm,
                              qk_norm_rope_kv_write_fp8=_qk_norm_rope_kv_write_fp8, swiglu=_swiglu,
                              sample_tokens=_sample_tokens, feed_tokens=_feed_tokens)


def embedding(out, table, ids) -> None:
    """out [T, D] = table[ids] for 16-bit tables (model/model_architecture.cpp:149)."""
    if ids.numel() == 0:
        return
    _require_cuda(out, table, ids)
    check("embedding", _lib.lib().cvh_embedding(out.data_ptr(), table.data_ptr(), ids.data_ptr(), ids.numel(),
                                                table.size(1), table.size(0), _stream(out)))


def build_token_metadata(cu_seqlens, positions, block_tables, block_size: int):
    """(token_seq, slot_mapping, token_kv_len) for a ragged batch (model/model_architecture.cpp:137-147)."""
    T = positions.size(0)
    S = cu_seqlens.size(0) - 1
    _require_cuda(cu_seqlens, positions, block_tables)
    dev = positions.device
    seq = torch.empty(T, dtype=torch.int64, device=dev)
    slot = torch.empty(T, dtype=torch.int64, device=dev)
    kvl = torch.empty(T, dtype=torch.int64, device=dev)
    if T == 0:
        return seq, slot, kvl
    code = _lib.lib().cvh_build_token_metadata(cu_seqlens.data_ptr(), S, positions.data_ptr(), T,
                                               block_tables.data_ptr(), block_tables.size(1), int(block_size),
                                               seq.data_ptr(), slot.data_ptr(), kvl.data_ptr(), _stream(positions))
    check("build_token_metadata", code)
    return seq, slot, kvl


def rope_tables(max_position: int, head_dim: int, theta: float):
    """Host float32 cos/sin tables [max_position, head_dim/2] (model/model_architecture.cpp:67-75)."""
    cos = torch.empty(max_position, head_dim // 2, dtype=torch.float32)
    sin = torch.empty_like(cos)
    check("rope_tables", _lib.lib().cvh_rope_tables_host(cos.data_ptr(), sin.data_ptr(), max_position, head_dim,
                                                         float(theta)))
    return cos, sin


def fp8_e4m3_quantize(dst, src, inv_scale: float) -> None:
    _require_cuda(dst, src)
    check("fp8_e4m3_quantize", _lib.lib().cvh_fp8_e4m3_quantize(dst.data_ptr(), src.data_ptr(), src.numel(),
                                                                 float(inv_scale), _stream(src)))


def gemm_supported(n: int, k: int) -> bool:
    """Shapes cvh_gemm_bf16_nt takes: N % 16 == 0 and K % 128 == 0."""
    return n % 16 == 0 and k % 128 == 0


def linear(out, x, w, config: int = 0) -> None:
    """out [M, N] = x [M, K] . w [N, K]^T in bf16 with fp32 accumulation (at::linear of the layer
    loop, model/model_architecture.cpp:155,178,182,185,224) on the gfx950 MFMA GEMM."""
    M = x.size(0)
    if M == 0:
        return
    _require_cuda(out, x, w)
    if not (x.dtype == w.dtype == out.dtype == torch.bfloat16):
        raise ValueError("linear: bf16 tensors only")
    N, K = w.shape
    if x.size(1) != K or tuple(out.shape) != (M, N):
        raise ValueError(f"linear: shapes x {tuple(x.shape)}, w {tuple(w.shape)}, out {tuple(out.shape)}")
    check("gemm_bf16_nt", _lib.lib().cvh_gemm_bf16_nt(out.data_ptr(), x.data_ptr(), w.data_ptr(), M, N, K,
                                                      int(config), _stream(out)))


FUSED_RESIDUAL, FUSED_SWIGLU_ROWNORM, FUSED_QKV = 0, 1, 2


def row_ss_slots(n: int) -> int:
    """Partial sums of squares per row that linear_residual writes for an N-wide row (N / 16)."""
    return n // 16


def linear_residual(resid, row_ss, x, w, config: int = 0) -> None:
    """resid [M, N] <- bf16(resid + bf16(x . w^T)) (the residual add of add_rms_norm,
    kernels/fused_ops.cu:70-73, in the projection's epilogue) and row_ss [M, N/16] <- the new
    residual's sum of squares per 16 columns, which a *_rownorm projection turns into the row's
    RMSNorm factor."""
    M = x.size(0)
    if M == 0:
        return
    _require_cuda(resid, row_ss, x, w)
    N, K = w.shape
    if tuple(resid.shape) != (M, N) or x.size(1) != K or tuple(row_ss.shape) != (M, row_ss_slots(N)):
        raise ValueError(f"linear_residual: shapes resid {tuple(resid.shape)}, x {tuple(x.shape)}, w {tuple(w.shape)}, "
                         f"row_ss {tuple(row_ss.shape)}")
    if not (x.dtype == w.dtype == resid.dtype == torch.bfloat16 and row_ss.dtype == torch.float32):
        raise ValueError("linear_residual: bf16 tensors and a float32 row_ss")
    check("gemm_bf16_nt_residual", _lib.lib().cvh_gemm_bf16_nt_residual(
        resid.data_ptr(), row_ss.data_ptr(), x.data_ptr(), w.data_ptr(), M, N, K, int(config), _stream(x)))


def fold_norm_gain(w, gain) -> torch.Tensor:
    """w' = bf16(w * gain) over the input columns: the weight a *_rownorm projection takes for an
    RMSNorm with that gain."""
    return (w.float() * gain.float()[None, :]).to(torch.bfloat16)


def linear_swiglu_rownorm(act, x, row_ss, eps: float, w_folded, config: int = 0) -> None:
    """act [M, I] = swiglu(rms(x) . w^T) with x the raw residual rows, rms's factor from row_ss
    (linear_residual) and its gain folded into w (fold_norm_gain of the 16-row interleaved gate/up
    weight)."""
    M = x.size(0)
    if M == 0:
        return
    _require_cuda(act, x, row_ss, w_folded)
    N, K = w_folded.shape
    if x.size(1) != K or tuple(act.shape) != (M, N // 2) or tuple(row_ss.shape) != (M, row_ss_slots(K)):
        raise ValueError("linear_swiglu_rownorm: shapes")
    check("gemm_bf16_nt_swiglu_rownorm", _lib.lib().cvh_gemm_bf16_nt_swiglu_rownorm(
        act.data_ptr(), x.data_ptr(), row_ss.data_ptr(), float(eps), w_folded.data_ptr(), M, N // 2, K, int(config),
        _stream(x)))


def qkv_norm_rope_kv_write_fp8(q_out, x, row_ss, x_eps: float, w_qkv, q_norm, k_norm, cos, sin, positions, slots,
                               k_cache, v_cache, k_scale, v_scale, n_heads: int, n_kv_heads: int, eps: float,
                               config: int = 0) -> None:
    """The QKV projection with qk_norm_rope_kv_write_fp8 in its epilogue: q_out [T, H, HD] and the
    K/V cache writes of fused.qk_norm_rope_kv_write_fp8 over qkv = x . w_qkv^T, without the qkv
    tensor. row_ss None: x is the normed input as is; else x is the raw residual, normed by the
    factor row_ss gives, with the norm gain folded into w_qkv (fold_norm_gain)."""
    T = x.size(0)
    if T == 0:
        return
    _require_cuda(q_out, x, row_ss, w_qkv, q_norm, k_norm, cos, sin, positions, slots, k_cache, v_cache, k_scale,
                  v_scale)
    N, D = w_qkv.shape
    HD = q_out.size(2)
    if x.size(1) != D or N != (n_heads + 2 * n_kv_heads) * HD or tuple(q_out.shape[:2]) != (T, n_heads):
        raise ValueError("qkv_norm_rope_kv_write_fp8: shapes")
    if row_ss is not None and tuple(row_ss.shape) != (T, row_ss_slots(D)):
        raise ValueError("qkv_norm_rope_kv_write_fp8: row_ss shape")
    check("gemm_qkv_norm_rope_kv_write_fp8", _lib.lib().cvh_gemm_qkv_norm_rope_kv_write_fp8(
        q_out.data_ptr(), x.data_ptr(), _ptr(row_ss), float(x_eps), w_qkv.data_ptr(), q_norm.data_ptr(),
        k_norm.data_ptr(), cos.data_ptr(), sin.data_ptr(), positions.data_ptr(), slots.data_ptr(), k_cache.data_ptr(),
        v_cache.data_ptr(), k_scale.data_ptr(), v_scale.data_ptr(), T, D, int(n_heads), int(n_kv_heads), HD,
        k_cache.size(1), _scale_mode(k_scale), float(eps), int(config), _stream(x)))


def interleave_gate_up(w_gate_up: torch.Tensor) -> torch.Tensor:
    """[2I, K] gate-then-up weight rows -> the 16-row interleaved layout linear_swiglu takes."""
    n, k = w_gate_up.shape
    i = n // 2
    if n % 32:
        raise ValueError("interleave_gate_up: 2I must be a multiple of 32")
    return w_gate_up.view(2, i // 16, 16, k).transpose(0, 1).reshape(n, k).contiguous()


def deinterleave_gate_up(w: torch.Tensor) -> torch.Tensor:
    """Inverse of interleave_gate_up: interleaved [2I, K] rows -> gate rows then up rows."""
    n, k = w.shape
    return w.view(n // 32, 2, 16, k).transpose(0, 1).reshape(n, k).contiguous()


def linear_swiglu(act, x, w_interleaved, config: int = 0) -> None:
    """act [M, I] = swiglu(x . w^T) with w's gate/up rows interleaved by 16 (at::linear +
    fused::swiglu, model/model_architecture.cpp:182-184) in one gfx950 kernel."""
    M = x.size(0)
    if M == 0:
        return
    _require_cuda(act, x, w_interleaved)
    if not (x.dtype == w_interleaved.dtype == act.dtype == torch.bfloat16):
        raise ValueError("linear_swiglu: bf16 tensors only")
    N, K = w_interleaved.shape
    if x.size(1) != K or tuple(act.shape) != (M, N // 2):
        raise ValueError(f"linear_swiglu: shapes x {tuple(x.shape)}, w {tuple(w_interleaved.shape)}, act {tuple(act.shape)}")
    check("gemm_bf16_nt_swiglu", _lib.lib().cvh_gemm_bf16_nt_swiglu(act.data_ptr(), x.data_ptr(), w_interleaved.data_ptr(),
                                                                    M, N // 2, K, int(config), _stream(act)))
