"""Qwen3 model runner on the gfx950 kernels: paged FP8 KV cache, eager ragged steps and
HIP-graph-captured decode steps.

Mirrors the reference's runner/model split:
  * ``Qwen3.forward``      — Qwen3::forward_backbone + compute_logits
                             (model/model_architecture.cpp:130-191,222-236): every op is a HIP
                             kernel of this package (embedding, norms, QK-norm/RoPE/FP8 cache write,
                             paged attention, SwiGLU, sampler, and the four projections through the
                             gfx950 GEMM for batches of up to 256 rows, which covers every decode
                             graph); prompt batches above that and the tied lm_head above 64 rows
                             use hipBLASLt through torch, which is faster there.
  * ``KVCache``            — ModelRunner::bind_cache layout (engine/model_runner.cpp:104-113):
                             K/V uint8 [L][NB+1][BS][KV][HD], scales f32 [L][NB+1][KV][BS]; block NB
                             is the scratch block that idle graph rows write to (:69,:346).
  * ``ModelRunner.run``    — ModelRunner::launch/collect (:169-212): decode rows go to the native
                             decode runner (include/cppvllm_runner.h, csrc/decode_runner.cpp), which
                             replays its HIP graph of the smallest batch size >= the row count
                             (:414-428; sizes 1,2,4,8,16,32,...,max as :380-383); the other rows
                             run one eager ragged forward (fresh prefills and continuations share
                             the paged path).
Weights are random N(0, std) bf16 (no checkpoint is loaded); norm gains are 1.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F

from . import _lib, ops

fused = ops.fused

# Row counts up to which cvh_gemm_bf16_nt is faster than hipBLASLt on MI355X (measured over the
# Qwen3-0.6B projection shapes and the tied lm_head).
GEMM_MAX_ROWS = 256
LM_HEAD_MAX_ROWS = 64
# Row counts from which the projections with fused layer-boundary epilogues (residual add + norm
# partials, row-normed inputs, QK-norm/RoPE/KV write) beat the projection + standalone-kernel
# sequence (measured per decode layer on MI355X: 16 rows 35.2 -> 34.8 us, 96 rows 43.8 -> 36.9,
# 256 rows 50.1 -> 44.3; at 1 row 31.4 -> 33.8).
FUSED_MIN_ROWS = 16


def _linear(x, w, max_rows: int = GEMM_MAX_ROWS):
    """x [M, K] . w[N, K]^T in bf16 (at::linear)."""
    if x.size(0) <= max_rows and ops.gemm_supported(*w.shape):
        y = torch.empty((x.size(0), w.size(0)), dtype=x.dtype, device=x.device)
        ops.linear(y, x, w)
        return y
    return F.linear(x, w)


@dataclass
class Qwen3Config:
    """Qwen3-0.6B shape (config.h:12-25)."""
    dim: int = 1024
    n_layers: int = 28
    n_heads: int = 16
    n_kv_heads: int = 8
    head_dim: int = 128
    intermediate_size: int = 3072
    vocab_size: int = 151936
    norm_eps: float = 1e-6
    rope_theta: float = 1e6
    max_seq_len: int = 40960


class KVCache:
    """Per-layer FP8 paged cache (+1 scratch block at index num_blocks)."""

    def __init__(self, cfg: Qwen3Config, num_blocks: int, block_size: int, device):
        L, KV, HD = cfg.n_layers, cfg.n_kv_heads, cfg.head_dim
        nb = num_blocks + 1
        self.num_blocks, self.block_size, self.scratch_block = num_blocks, block_size, num_blocks
        self.k = torch.zeros((L, nb, block_size, KV, HD), dtype=torch.uint8, device=device)
        self.v = torch.zeros_like(self.k)
        self.ks = torch.zeros((L, nb, KV, block_size), dtype=torch.float32, device=device)
        self.vs = torch.zeros_like(self.ks)
        # per-layer views, made once (the kernels take [NB, BS, KV, HD] and [NB, KV, BS] per layer)
        self.layers = [(self.k[i], self.v[i], self.ks[i], self.vs[i]) for i in range(L)]

    @staticmethod
    def bytes_per_block(cfg: Qwen3Config, block_size: int) -> int:
        return 2 * cfg.n_layers * block_size * cfg.n_kv_heads * (cfg.head_dim + 4)


class Qwen3:
    """Random-init Qwen3 weights on the device and the forward pass over a ragged batch."""

    def __init__(self, cfg: Qwen3Config, device, seed: int = 0, std: float = 0.02):
        self.cfg = c = cfg
        self.device = device
        gen = torch.Generator(device=device).manual_seed(seed)
        bf16 = torch.bfloat16

        def rnd(*shape):
            return (torch.randn(shape, generator=gen, device=device) * std).to(bf16)

        H, KV, HD, D, I, L = c.n_heads, c.n_kv_heads, c.head_dim, c.dim, c.intermediate_size, c.n_layers
        self.embed = rnd(c.vocab_size, D)        # tied lm_head (config.h:24)
        self.wqkv = [rnd((H + 2 * KV) * HD, D) for _ in range(L)]
        self.wo = [rnd(D, H * HD) for _ in range(L)]
        # gate/up rows are stored interleaved in blocks of 16 (ops.interleave_gate_up) so that one
        # kernel computes the projection and the SwiGLU (batches of up to GEMM_MAX_ROWS rows); the
        # reference layout (gate rows, then up rows) is kept too, for the hipBLASLt projection of
        # prompt batches, whose output then goes to the SwiGLU kernel without a de-interleave copy
        # (+12.6 MB per layer at Qwen3-0.6B)
        self.gate_up_interleaved = (2 * I) % 32 == 0
        self.w_gate_up = [rnd(2 * I, D) for _ in range(L)]
        self.w_gu = [ops.interleave_gate_up(w) for w in self.w_gate_up] if self.gate_up_interleaved \
            else self.w_gate_up
        self.w_down = [rnd(D, I) for _ in range(L)]
        ones = lambda n: torch.ones(n, dtype=bf16, device=device)  # noqa: E731
        self.attn_norm = [ones(D) for _ in range(L)]
        self.ffn_norm = [ones(D) for _ in range(L)]
        self.q_norm = [ones(HD) for _ in range(L)]
        self.k_norm = [ones(HD) for _ in range(L)]
        self.final_norm = ones(D)
        cos, sin = ops.rope_tables(c.max_seq_len, HD, c.rope_theta)
        self.cos, self.sin = cos.to(device), sin.to(device)
        self.scale = 1.0 / math.sqrt(HD)
        self.unit_gain = ones(D)
        # False: every batch uses the reference's rounding points (normed input rounded to bf16, then
        # the gain, then the projection); True: batches of FUSED_MIN_ROWS..GEMM_MAX_ROWS rows take the
        # fused-epilogue projections, which round the gain-scaled weights instead
        self.fused_epilogues = True
        self.fold_gains()

    def fold_gains(self) -> None:
        """Weights of the fused decode path: the input norms' gains multiplied into the columns of
        the projections they feed (ops.fold_norm_gain; the same tensor where the gain is all ones).
        Call again after changing attn_norm / ffn_norm."""
        c = self.cfg
        # the gate/up row-normed tile above 128 rows is 128 columns wide, so 2I must be a multiple of 128
        self.fused_ok = (c.head_dim == 128 and c.dim % 256 == 0 and c.dim <= 1024 and self.gate_up_interleaved
                         and (2 * c.intermediate_size) % 128 == 0)
        fold = lambda w, gain: w if bool((gain == 1).all()) else ops.fold_norm_gain(w, gain)  # noqa: E731
        self.wqkv_f = [fold(w, g) for w, g in zip(self.wqkv, self.attn_norm)]
        self.w_gu_f = [fold(w, g) for w, g in zip(self.w_gu, self.ffn_norm)] if self.fused_ok else []

    def forward(self, cache: KVCache, tokens, positions, cu_seqlens, block_tables, workspace, planned: bool,
                shared_blocks=None):
        """Backbone over T ragged tokens; returns the final-normed hidden rows x [T, D]
        (the last layer's add_rms_norm applies the final norm: resid + mlp, then RMSNorm, as
        h.add_(mlp) + rms_norm(h, final_norm) at model_architecture.cpp:188,224)."""
        c = self.cfg
        T = tokens.numel()
        H, KV, HD, D, I = c.n_heads, c.n_kv_heads, c.head_dim, c.dim, c.intermediate_size
        dev, bf16, eps = self.device, torch.bfloat16, c.norm_eps
        seq, slot, kvl = ops.build_token_metadata(cu_seqlens, positions, block_tables, cache.block_size)
        h = torch.empty((T, D), dtype=bf16, device=dev)
        ops.embedding(h, self.embed, tokens)
        x = torch.empty_like(h)
        shared = planned and shared_blocks is not None
        if planned:   # shared_blocks: per-row leading blocks shared with other rows (shared-prefix units)
            ops.paged_attention_plan(block_tables, seq, kvl, H, KV, HD, cache.block_size, workspace,
                                     shared_blocks=shared_blocks if shared else None)
        q = torch.empty((T, H, HD), dtype=bf16, device=dev)
        att = torch.empty_like(q)
        act = torch.empty((T, I), dtype=bf16, device=dev)
        # prompt / chunked-prefill batches (several tokens per sequence on average) take the MFMA
        # multi-query kernel; decode rows take the stream-K decode kernel
        S = cu_seqlens.numel() - 1
        multi_query = not planned and T >= 2 * S and ops.prefill_supported(H, KV, HD)
        if multi_query:   # the 64-token groups longest key walk first, once for all layers
            pws = ops.prefill_workspace(T, dev)
            ops.paged_attention_prefill_plan(seq, kvl, block_tables.size(1), cache.block_size, pws)

        def attention(li, kc, vc, ks, vs):
            if multi_query:
                ops.paged_attention_fp8_prefill(att, q, kc, vc, ks, vs, block_tables, seq, kvl, self.scale,
                                                workspace=pws)
            else:
                ops.paged_attention_fp8(att, q, kc, vc, ks, vs, block_tables, seq, kvl, self.scale,
                                        workspace=workspace, planned=planned, shared=shared)

        if self.fused_ok and self.fused_epilogues and FUSED_MIN_ROWS <= T <= GEMM_MAX_ROWS:
            # Layer boundaries in the projections' epilogues: o_proj / down_proj add into the
            # residual h and leave its per-16-column sums of squares in ss; qkv / gate-up take h
            # raw and apply the row's RMS factor from ss (gains folded into their weights); qkv
            # runs the QK-norm / RoPE / FP8 K/V write on its own output tile. Layer 0's input is
            # normed with a unit gain.
            ss = torch.empty((T, ops.row_ss_slots(D)), dtype=torch.float32, device=dev)
            fused.rms_norm(x, h, self.unit_gain, eps)
            for li in range(c.n_layers):
                kc, vc, ks, vs = cache.layers[li]
                ops.qkv_norm_rope_kv_write_fp8(q, x if li == 0 else h, None if li == 0 else ss, eps, self.wqkv_f[li],
                                               self.q_norm[li], self.k_norm[li], self.cos, self.sin, positions, slot,
                                               kc, vc, ks, vs, H, KV, eps)
                attention(li, kc, vc, ks, vs)
                ops.linear_residual(h, ss, att.view(T, H * HD), self.wo[li])
                ops.linear_swiglu_rownorm(act, h, ss, eps, self.w_gu_f[li])
                ops.linear_residual(h, ss, act, self.w_down[li])
            fused.rms_norm(x, h, self.final_norm, eps)
            return x

        fused.rms_norm(x, h, self.attn_norm[0], eps)
        for li in range(c.n_layers):
            kc, vc, ks, vs = cache.layers[li]
            qkv = _linear(x, self.wqkv[li])
            fused.qk_norm_rope_kv_write_fp8(q, qkv, self.q_norm[li], self.k_norm[li], self.cos, self.sin, positions,
                                            slot, kc, vc, ks, vs, None, None, H, KV, eps)
            attention(li, kc, vc, ks, vs)
            o = _linear(att.view(T, H * HD), self.wo[li])
            fused.add_rms_norm(h, o, self.ffn_norm[li], x, eps)
            if self.gate_up_interleaved and T <= GEMM_MAX_ROWS and ops.gemm_supported(2 * I, D):
                ops.linear_swiglu(act, x, self.w_gu[li])
            else:
                fused.swiglu(act, _linear(x, self.w_gate_up[li]))
            m = _linear(act, self.w_down[li])
            nxt = self.attn_norm[li + 1] if li + 1 < c.n_layers else self.final_norm
            fused.add_rms_norm(h, m, nxt, x, eps)
        return x

    def sample(self, x_rows, out, temps=None, seed: int = 0, offset: int = 0) -> None:
        """Next token of each row (compute_logits + sample_tokens, model_architecture.cpp:222-226,
        model_runner.cpp:262-272): greedy where temps is None or <= 0, else Gumbel-max. Logits
        stay bf16: the reference's float copy of them holds the same values."""
        logits = _linear(x_rows.contiguous(), self.embed, LM_HEAD_MAX_ROWS)
        fused.sample_tokens(out, logits, None, temps, seed, offset)


def _graph_sizes(max_batch: int) -> list[int]:
    """1, 2, 4, 8, then multiples of 16, then max (model_runner.cpp:380-383)."""
    s = [b for b in (1, 2, 4, 8) if b < max_batch]
    s += list(range(16, max_batch, 16))
    s.append(max_batch)
    return s


class _Graph:
    """A decode graph of the native runner, replayed on torch's current stream."""

    def __init__(self, runner: "ModelRunner", batch: int, shared: bool):
        self.runner, self.batch, self.shared = runner, batch, shared

    def replay(self) -> None:
        r = self.runner
        ops.check("runner_replay", r._L.cvh_runner_replay(r._handle, self.batch, int(self.shared),
                                                           torch.cuda.current_stream().cuda_stream))


class ModelRunner:
    """Launches scheduled batches (cppvllm_amd.engine_core.Batch) asynchronously and collects one
    sampled token per row (-1 for rows that do not sample).

    Decode rows run in the native decode runner (include/cppvllm_runner.h): it stages the rows
    through pinned memory, runs the 28-layer forward through the library's C ABI and captures /
    replays it as HIP graphs with the HIP runtime (engine/model_runner.cpp:327-428); this class
    hands it the weights' and the cache's device pointers and samples its output rows. Rows that
    are not plain decode rows (fresh prompts, chunked-prefill continuations) run one eager ragged
    forward of Qwen3.forward.

    Two launch slots alternate (the reference's two-deep ring, engine/model_runner.cpp:169-212 and
    engine/llm_engine.cpp:70-113): each slot owns pinned host staging and a device buffer of the
    step's sampled tokens in row order, so step N+1 can be staged and launched while step N runs,
    reading N's samples on the device (cvh_feed_tokens) for the tokens the scheduler left as
    placeholders. Device input buffers are shared by the slots: the stream orders their reuse.
    A slot is reused two launches later, after collect() of its previous step has synchronised on
    that step's completion event."""

    def __init__(self, model: Qwen3, cache: KVCache, *, max_num_batched_tokens: int = 4096, max_num_seqs: int = 256,
                 max_model_len: int = 4096, graph_max_blocks: int | None = None, enforce_eager: bool = False,
                 seed: int = 0):
        self.model, self.cache = model, cache
        c = model.cfg
        dev = model.device
        BS = cache.block_size
        self.max_tokens = Tm = max(max_num_batched_tokens, max_num_seqs)
        self.max_seqs = Sm = max_num_seqs
        self.table_width = Wm = -(-max_model_len // BS)
        self.graph_width = graph_max_blocks or self.table_width
        self.max_graph_batch = max_num_seqs
        if self.max_graph_batch > GEMM_MAX_ROWS:
            raise ValueError(f"max_num_seqs {max_num_seqs} > {GEMM_MAX_ROWS} (decode graph rows)")
        i64 = dict(dtype=torch.int64)
        # eager inputs: tok | pos | feed | cu | sampled token rows | their batch rows | tables (S x W)
        self.e_off = np.cumsum([0, Tm, Tm, Tm, Sm + 1, Sm, Sm]).tolist()
        self.e_len = self.e_off[-1] + Sm * Wm
        self.d_earena = torch.zeros(self.e_len, device=dev, **i64)
        # per launch slot: pinned staging (StagedBuffer, utils/tensor.h:64-110), sampled tokens
        self.h_earena = [torch.zeros(self.e_len, pin_memory=True, **i64) for _ in range(2)]
        self.h_temps = [torch.zeros(Sm, pin_memory=True, dtype=torch.float32) for _ in range(2)]
        self.d_temps = torch.zeros(Sm, device=dev, dtype=torch.float32)
        self.d_sampled = [torch.zeros(Sm, device=dev, **i64) for _ in range(2)]
        self.h_sampled = [torch.zeros(Sm, pin_memory=True, **i64) for _ in range(2)]
        self.d_tmp = torch.zeros(Sm, device=dev, **i64)
        self.events = [torch.cuda.Event() for _ in range(2)]
        self.slot, self.last_slot = 0, None
        self.seed, self.sample_step = seed, 0
        self.ws_eager = ops.paged_attention_workspace(Tm, c.n_heads, c.n_kv_heads, c.head_dim, Wm, BS, 0, dev)
        self.graphs: dict[int, _Graph] = {}
        self.graphs_shared: dict[int, _Graph] = {}
        self.shared_replays = 0
        # decode graph replays and the keys their real rows attend over (for per-launch byte counts)
        self.decode_replays = 0
        self.decode_rows = 0
        self.decode_keys = 0
        # decode rows: padded to a batch size of _graph_sizes, planned attention (a replay and an
        # eager run of a decode step give the same bits)
        self.graph_sizes = _graph_sizes(self.max_graph_batch)
        self.g_hidden = torch.empty((self.graph_sizes[-1], c.dim), dtype=torch.bfloat16, device=dev)
        self._L = _lib.lib()
        self._handle = None
        self._create_native()
        if not enforce_eager:
            self.capture_graphs()
        self.warm_sampler()

    # ---- the native decode runner ----------------------------------------------------------------
    def _create_native(self) -> None:
        """Describe the model and cache to cvh_runner_create. The runner keeps the device pointers:
        the tensors are referenced here for its lifetime (call again after replacing weights)."""
        m, c, cache = self.model, self.model.cfg, self.cache
        fused = m.fused_ok and m.fused_epilogues
        layers = (_lib.RunnerLayer * c.n_layers)()
        keep = []
        for li in range(c.n_layers):
            kc, vc, ks, vs = cache.layers[li]
            ts = dict(w_qkv=m.wqkv[li], w_qkv_folded=m.wqkv_f[li], w_o=m.wo[li], w_gate_up=m.w_gu[li],
                      w_gate_up_folded=m.w_gu_f[li] if fused else None, w_down=m.w_down[li],
                      attn_norm=m.attn_norm[li], ffn_norm=m.ffn_norm[li], q_norm=m.q_norm[li], k_norm=m.k_norm[li],
                      k_cache=kc, v_cache=vc, k_scale=ks, v_scale=vs)
            for k, t in ts.items():
                if t is not None:
                    if not t.is_contiguous():
                        raise ValueError(f"runner: {k} of layer {li} is not contiguous")
                    keep.append(t)
                setattr(layers[li], k, None if t is None else t.data_ptr())
        if not m.gate_up_interleaved:
            raise ValueError("runner: the decode graphs need gate/up rows interleaved by 16 (2I % 32 == 0)")
        desc = _lib.RunnerDesc(
            n_layers=c.n_layers, dim=c.dim, n_heads=c.n_heads, n_kv_heads=c.n_kv_heads, head_dim=c.head_dim,
            intermediate=c.intermediate_size, vocab=c.vocab_size, norm_eps=c.norm_eps, attn_scale=m.scale,
            block_size=cache.block_size, scale_mode=_lib.SCALE_PER_TOKEN_HEAD, max_batch=self.graph_sizes[-1],
            table_width=self.graph_width, scratch_block=cache.scratch_block,
            fused_min_rows=FUSED_MIN_ROWS if fused else 1, fused_max_rows=GEMM_MAX_ROWS if fused else 0,
            embed=m.embed.data_ptr(), final_norm=m.final_norm.data_ptr(), unit_gain=m.unit_gain.data_ptr(),
            rope_cos=m.cos.data_ptr(), rope_sin=m.sin.data_ptr(), hidden=self.g_hidden.data_ptr(), layers=layers)
        keep += [m.embed, m.final_norm, m.unit_gain, m.cos, m.sin, self.g_hidden]
        self.close()
        h = C.c_void_p()
        torch.cuda.synchronize()
        ops.check("runner_create", self._L.cvh_runner_create(C.byref(desc), C.byref(h)))
        self._handle, self._keep = h, keep
        self.graphs.clear()
        self.graphs_shared.clear()

    def close(self) -> None:
        """Free the native runner (its graphs, inputs and activations)."""
        if getattr(self, "_handle", None) is not None:
            torch.cuda.synchronize()
            self._L.cvh_runner_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _stage_graph_rows(self, toks, pos, tables, B: int, feed=None, slot: int = 0, shared=None) -> None:
        """Rows [0, S) are the decode rows; [S, B) are idle rows on the scratch block at position 0
        with kv_len 1 (model_runner.cpp:327-357). One host-to-device copy, then the feed of tokens
        from the previous step's samples where feed >= 0 (cvh_runner_stage)."""
        S = len(toks)
        i64 = lambda a: np.ascontiguousarray(a, dtype=np.int64)  # noqa: E731
        t, p = i64(toks), i64(pos)
        tab = i64(tables) if S else np.zeros((0, 1), np.int64)
        f = i64(feed) if feed is not None and S else None
        sh = np.ascontiguousarray(shared, dtype=np.int32) if shared is not None and S else None
        prev = None
        if f is not None and bool((f >= 0).any()):
            prev = self._prev_sampled().data_ptr()
        ptr = lambda a: None if a is None else a.ctypes.data  # noqa: E731
        ops.check("runner_stage", self._L.cvh_runner_stage(
            self._handle, slot, S, B, ptr(t), ptr(p), ptr(tab), tab.shape[1] if tab.ndim == 2 else 1, ptr(f), ptr(sh),
            prev, torch.cuda.current_stream().cuda_stream))

    def decode_eager(self, B: int, shared: bool = False) -> None:
        """The decode forward of the staged rows, launched eagerly (the body the graphs hold)."""
        ops.check("runner_forward", self._L.cvh_runner_forward(self._handle, B, int(shared),
                                                                torch.cuda.current_stream().cuda_stream))

    def capture_graphs(self) -> None:
        """One graph per batch size of _graph_sizes, plain and shared-prefix variants (captured by
        the native runner on its own stream; model_runner.cpp:371-405)."""
        empty = np.zeros((0, self.graph_width), dtype=np.int64)
        torch.cuda.synchronize()
        for shared, dst in ((False, self.graphs), (True, self.graphs_shared)):
            for B in reversed(self.graph_sizes):
                self._stage_graph_rows([], [], empty, B)
                torch.cuda.synchronize()
                ops.check("runner_capture", self._L.cvh_runner_capture(self._handle, B, int(shared)))
                dst[B] = _Graph(self, B, shared)
        torch.cuda.synchronize()

    def warm_sampler(self) -> None:
        """Run the lm_head + sampler once per row count above LM_HEAD_MAX_ROWS (up to the
        sequence cap) at start-up: hipBLASLt picks its algorithm on the first call of each shape,
        which inside a run costs ~0.15 s over config 5's decode batch sizes."""
        c = self.model.cfg
        dev = self.model.device
        for S in range(LM_HEAD_MAX_ROWS + 1, self.max_seqs + 1):
            self.model.sample(torch.zeros((S, c.dim), dtype=torch.bfloat16, device=dev), self.d_tmp[:S])
        torch.cuda.synchronize()

    # ---- sampling --------------------------------------------------------------------------------
    def _sample(self, x_rows, out, temps_dev) -> None:
        self.model.sample(x_rows, out, temps_dev, self.seed, self.sample_step)
        self.sample_step += 1

    def _prev_sampled(self):
        if self.last_slot is None:
            raise RuntimeError("a batch feeds tokens but no step was launched before it")
        return self.d_sampled[self.last_slot]

    # ---- eager ragged forward ------------------------------------------------------------------
    def _run_eager(self, toks, pos, cu, tables, sample_rows, temps_dev, feed=None, slot: int = 0, row_ids=None,
                   out=None):
        """One eager forward over a ragged batch; samples the token rows `sample_rows` into
        out[row_ids] (row_ids: numpy batch rows), or into a temporary that is returned."""
        T, S = len(toks), len(cu) - 1
        W = tables.shape[1]
        if T > self.max_tokens or S > self.max_seqs or W > self.table_width:
            raise ValueError(f"batch exceeds the runner's limits (T={T}, S={S}, W={W})")
        R = len(sample_rows)
        o = self.e_off
        h = self.h_earena[slot].numpy()
        h[o[0]:o[0] + T], h[o[1]:o[1] + T] = toks, pos
        need_feed = feed is not None and bool((feed >= 0).any())
        if need_feed:
            h[o[2]:o[2] + T] = feed
        h[o[3]:o[3] + S + 1] = cu
        h[o[4]:o[4] + R] = sample_rows
        if row_ids is not None:
            h[o[5]:o[5] + R] = row_ids
        h[o[6]:o[6] + S * W] = tables.reshape(-1)
        n = o[6] + S * W
        self.d_earena[:n].copy_(self.h_earena[slot][:n], non_blocking=True)
        d = self.d_earena
        tok = d[o[0]:o[0] + T]
        if need_feed:
            fused.feed_tokens(tok, d[o[2]:o[2] + T], self._prev_sampled())
        x = self.model.forward(self.cache, tok, d[o[1]:o[1] + T], d[o[3]:o[3] + S + 1],
                               d[o[6]:o[6] + S * W].view(S, W), self.ws_eager, planned=False)
        if R == 0:
            return self.d_tmp[:0]
        rows = x.index_select(0, d[o[4]:o[4] + R])
        self._sample(rows, self.d_tmp[:R], temps_dev)
        if out is not None and row_ids is not None:
            out.index_copy_(0, d[o[5]:o[5] + R], self.d_tmp[:R])
        return self.d_tmp[:R]

    # ---- one step ----------------------------------------------------------------------------------
    def launch(self, batch, temps: np.ndarray | None = None):
        """Stage and enqueue one step: decode rows through the captured graph of the smallest
        batch size >= their count, the other rows in one eager ragged forward. Returns a handle
        for collect(). temps: per-row sampling temperature (None or <= 0: greedy)."""
        slot = self.slot
        S = batch.num_seqs
        if S > self.max_seqs:
            raise ValueError(f"{S} rows > max_num_seqs {self.max_seqs}")
        d0, d1 = batch.group_start[0], batch.group_start[1]
        cu = batch.cu_seqlens
        feed = batch.feed_src
        use_graph = d1 > d0      # decode rows: a captured graph, or the same body run eagerly
        first_eager = d1 if use_graph else d0
        samp = np.nonzero(batch.samples[first_eager:])[0]
        # temperatures of the sampled rows: graph rows first, then the eager rows, one copy
        temps_dev_g = temps_dev_e = None
        if temps is not None and np.any(temps > 0):
            ht = self.h_temps[slot].numpy()
            ng = d1 - d0 if use_graph else 0
            if ng:
                ht[:ng] = temps[d0:d1]
            ht[ng:ng + len(samp)] = temps[first_eager + samp]
            self.d_temps[:ng + len(samp)].copy_(self.h_temps[slot][:ng + len(samp)], non_blocking=True)
            temps_dev_g = self.d_temps[:ng] if ng else None
            temps_dev_e = self.d_temps[ng:ng + len(samp)]
        out = self.d_sampled[slot]
        if use_graph:
            t0 = cu[d0:d1]
            n = d1 - d0
            B = next(b for b in self.graph_sizes if b >= n)
            shared = None if batch.shared_blocks is None else batch.shared_blocks[d0:d1]
            any_shared = shared is not None and bool((shared > 0).any())
            self._stage_graph_rows(batch.tokens[t0], batch.positions[t0], batch.block_tables[d0:d1], B,
                                   None if feed is None else feed[t0], slot, shared if any_shared else None)
            graphs = self.graphs_shared if any_shared else self.graphs
            if graphs:
                graphs[B].replay()
            else:
                self.decode_eager(B, any_shared)
            self.shared_replays += int(any_shared)
            self.decode_replays += 1
            self.decode_rows += n
            self.decode_keys += int(batch.positions[t0].sum()) + n
            self._sample(self.g_hidden[:n], out[d0:d1], temps_dev_g)
        if first_eager < S:
            a = first_eager
            t_lo, t_hi = cu[a], cu[S]
            rows_cu = cu[a:] - t_lo
            last_tok = rows_cu[samp + 1] - 1
            tables = batch.block_tables[a:]
            W = min(tables.shape[1], self.table_width)
            self._run_eager(batch.tokens[t_lo:t_hi], batch.positions[t_lo:t_hi], rows_cu, tables[:, :W], last_tok,
                            temps_dev_e, None if feed is None else feed[t_lo:t_hi], slot, a + samp, out)
        self.h_sampled[slot][:S].copy_(out[:S], non_blocking=True)
        self.events[slot].record()
        self.last_slot, self.slot = slot, slot ^ 1
        return (slot, S, batch.samples.copy())

    def collect(self, handle) -> np.ndarray:
        """Wait for a launched step and return its sampled token per row (-1 where none)."""
        slot, S, samples = handle
        self.events[slot].synchronize()
        vals = self.h_sampled[slot][:S].numpy().copy()
        vals[~samples] = -1
        return vals

    def run(self, batch, temps: np.ndarray | None = None) -> np.ndarray:
        """launch + collect (a synchronous step)."""
        return self.collect(self.launch(batch, temps))
