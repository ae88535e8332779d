"""Qwen3 model runner on the gfx950 kernels: paged FP8 KV cache, eager ragged steps and
HIP-graph-captured decode steps.

Mirrors the reference's runner/model split:
  * ``Qwen3.forward``      — Qwen3::forward_backbone + compute_logits
                             (model/model_architecture.cpp:130-191,222-236): every non-GEMM op is a
                             HIP kernel of this package (embedding, norms, QK-norm/RoPE/FP8 cache
                             write, paged attention, SwiGLU, sampler); the four projections and the
                             tied lm_head are hipBLASLt GEMMs through torch.
  * ``KVCache``            — ModelRunner::bind_cache layout (engine/model_runner.cpp:104-113):
                             K/V uint8 [L][NB+1][BS][KV][HD], scales f32 [L][NB+1][KV][BS]; block NB
                             is the scratch block that idle graph rows write to (:69,:346).
  * ``ModelRunner.run``    — ModelRunner::launch/collect (:169-212): decode rows replay a captured
                             graph of the smallest batch size >= the row count (:414-428; sizes
                             1,2,4,8,16,32,...,max as :380-383), the other rows run one eager
                             ragged forward (fresh prefills and continuations share the paged path).
Weights are random N(0, std) bf16 (no checkpoint is loaded); norm gains are 1.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F

from . import ops

fused = ops.fused


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
        self.w_gate_up = [rnd(2 * I, D) for _ in range(L)]
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

    def forward(self, cache: KVCache, tokens, positions, cu_seqlens, block_tables, workspace, planned: bool):
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
        fused.rms_norm(x, h, self.attn_norm[0], eps)
        if planned:
            ops.paged_attention_plan(block_tables, seq, kvl, H, KV, HD, cache.block_size, workspace)
        q = torch.empty((T, H, HD), dtype=bf16, device=dev)
        att = torch.empty_like(q)
        act = torch.empty((T, I), dtype=bf16, device=dev)
        # prompt / chunked-prefill batches (several tokens per sequence on average) take the MFMA
        # multi-query kernel; decode rows take the stream-K decode kernel
        S = cu_seqlens.numel() - 1
        multi_query = not planned and T >= 2 * S and ops.prefill_supported(H, KV, HD)
        for li in range(c.n_layers):
            kc, vc, ks, vs = cache.layers[li]
            qkv = F.linear(x, self.wqkv[li])
            fused.qk_norm_rope_kv_write_fp8(q, qkv, self.q_norm[li], self.k_norm[li], self.cos, self.sin, positions,
                                            slot, kc, vc, ks, vs, None, None, H, KV, eps)
            if multi_query:
                ops.paged_attention_fp8_prefill(att, q, kc, vc, ks, vs, block_tables, seq, kvl, self.scale)
            else:
                ops.paged_attention_fp8(att, q, kc, vc, ks, vs, block_tables, seq, kvl, self.scale,
                                        workspace=workspace, planned=planned)
            o = F.linear(att.view(T, H * HD), self.wo[li])
            fused.add_rms_norm(h, o, self.ffn_norm[li], x, eps)
            gu = F.linear(x, self.w_gate_up[li])
            fused.swiglu(act, gu)
            m = F.linear(act, self.w_down[li])
            nxt = self.attn_norm[li + 1] if li + 1 < c.n_layers else self.final_norm
            fused.add_rms_norm(h, m, nxt, x, eps)
        return x

    def sample(self, x_rows, out, temps=None, seed: int = 0, offset: int = 0) -> None:
        """Next token of each row (compute_logits + sample_tokens, model_architecture.cpp:222-226,
        model_runner.cpp:262-272): greedy where temps is None or <= 0, else Gumbel-max. Logits
        stay bf16: the reference's float copy of them holds the same values."""
        logits = F.linear(x_rows, self.embed)
        fused.sample_tokens(out, logits, None, temps, seed, offset)


def _graph_sizes(max_batch: int) -> list[int]:
    """1, 2, 4, 8, then multiples of 16, then max (model_runner.cpp:380-383)."""
    s = [b for b in (1, 2, 4, 8) if b < max_batch]
    s += list(range(16, max_batch, 16))
    s.append(max_batch)
    return s


class ModelRunner:
    """Runs scheduled batches (cppvllm_amd.engine_core.Batch) and returns one sampled token per
    row (-1 for rows that do not sample)."""

    def __init__(self, model: Qwen3, cache: KVCache, *, max_num_batched_tokens: int = 4096, max_num_seqs: int = 256,
                 max_model_len: int = 4096, graph_max_blocks: int | None = None, enforce_eager: bool = False,
                 seed: int = 0):
        self.model, self.cache = model, cache
        c = model.cfg
        dev = model.device
        BS = cache.block_size
        self.max_tokens = max(max_num_batched_tokens, max_num_seqs)
        self.max_seqs = max_num_seqs
        self.table_width = -(-max_model_len // BS)
        self.graph_width = graph_max_blocks or self.table_width
        i64 = dict(dtype=torch.int64)
        # pinned staging (StagedBuffer, utils/tensor.h:64-110) and device copies
        self.h_tok = torch.empty(self.max_tokens, pin_memory=True, **i64)
        self.h_pos = torch.empty(self.max_tokens, pin_memory=True, **i64)
        self.h_cu = torch.empty(self.max_seqs + 1, pin_memory=True, **i64)
        self.h_tab = torch.empty(self.max_seqs * max(self.table_width, self.graph_width), pin_memory=True, **i64)
        self.h_out = torch.empty(self.max_tokens, pin_memory=True, **i64)
        self.d_tok = torch.empty(self.max_tokens, device=dev, **i64)
        self.d_pos = torch.empty(self.max_tokens, device=dev, **i64)
        self.d_cu = torch.empty(self.max_seqs + 1, device=dev, **i64)
        self.d_tab = torch.empty(self.max_seqs * max(self.table_width, self.graph_width), device=dev, **i64)
        self.d_out = torch.empty(self.max_tokens, device=dev, **i64)
        self.d_rows = torch.empty(self.max_seqs, device=dev, **i64)
        self.h_rows = torch.empty(self.max_seqs, pin_memory=True, **i64)
        self.h_temps = torch.empty(self.max_seqs, pin_memory=True, dtype=torch.float32)
        self.d_temps = torch.empty(self.max_seqs, device=dev, dtype=torch.float32)
        self.seed, self.sample_step = seed, 0
        self.ws_eager = ops.paged_attention_workspace(self.max_tokens, c.n_heads, c.n_kv_heads, c.head_dim,
                                                      self.table_width, BS, 0, dev)
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self.max_graph_batch = max_num_seqs
        if not enforce_eager:
            self.capture_graphs()

    # ---- decode graphs -------------------------------------------------------------------------
    def _stage_graph_rows(self, toks, pos, tables, B: int) -> None:
        """Rows [0, S) are the decode rows; [S, B) are idle rows on the scratch block at position 0
        with kv_len 1 (model_runner.cpp:327-357)."""
        S = len(toks)
        Wg = self.graph_width
        ht, hp, hc = self.h_tok.numpy(), self.h_pos.numpy(), self.h_cu.numpy()
        tab = self.h_tab.numpy()[:B * Wg].reshape(B, Wg)
        ht[:S], hp[:S] = toks, pos
        ht[S:B], hp[S:B] = 0, 0
        hc[:B + 1] = np.arange(B + 1)
        tab[:] = -1
        if S:
            w = min(tables.shape[1], Wg)
            tab[:S, :w] = tables[:, :w]
        tab[S:B, 0] = self.cache.scratch_block
        self.d_tok[:B].copy_(self.h_tok[:B], non_blocking=True)
        self.d_pos[:B].copy_(self.h_pos[:B], non_blocking=True)
        self.d_cu[:B + 1].copy_(self.h_cu[:B + 1], non_blocking=True)
        self.d_tab[:B * Wg].copy_(self.h_tab[:B * Wg], non_blocking=True)

    def _graph_body(self, B: int, ws) -> None:
        Wg = self.graph_width
        x = self.model.forward(self.cache, self.d_tok[:B], self.d_pos[:B], self.d_cu[:B + 1],
                               self.d_tab[:B * Wg].view(B, Wg), ws, planned=True)
        self.g_hidden[:B].copy_(x)

    def capture_graphs(self) -> None:
        c = self.model.cfg
        sizes = _graph_sizes(self.max_graph_batch)
        Bmax = sizes[-1]
        self.ws_graph = ops.paged_attention_workspace(Bmax, c.n_heads, c.n_kv_heads, c.head_dim, self.graph_width,
                                                      self.cache.block_size, 0, self.model.device)
        self.g_hidden = torch.empty((Bmax, c.dim), dtype=torch.bfloat16, device=self.model.device)
        empty = np.zeros((0, self.graph_width), dtype=np.int64)
        self._stage_graph_rows([], [], empty, Bmax)
        torch.cuda.synchronize()
        pool = torch.cuda.graph_pool_handle()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for B in reversed(sizes):
                for _ in range(2):
                    self._graph_body(B, self.ws_graph)
                side.synchronize()
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, pool=pool, stream=side):
                    self._graph_body(B, self.ws_graph)
                self.graphs[B] = g
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()

    def _stage_temps(self, temps, n: int):
        if temps is None or not np.any(temps > 0):
            return None
        self.h_temps.numpy()[:n] = temps
        self.d_temps[:n].copy_(self.h_temps[:n], non_blocking=True)
        return self.d_temps[:n]

    def _sample(self, x_rows, temps) -> torch.Tensor:
        R = x_rows.size(0)
        self.model.sample(x_rows, self.d_out[:R], self._stage_temps(temps, R), self.seed, self.sample_step)
        self.sample_step += 1
        return self.d_out[:R]

    def _run_graph(self, toks, pos, tables, temps) -> torch.Tensor:
        S = len(toks)
        B = next(b for b in sorted(self.graphs) if b >= S)
        self._stage_graph_rows(toks, pos, tables, B)
        self.graphs[B].replay()
        return self._sample(self.g_hidden[:S], temps)

    # ---- eager ragged forward ------------------------------------------------------------------
    def _run_eager(self, toks, pos, cu, tables, sample_rows, temps) -> torch.Tensor:
        T, S = len(toks), len(cu) - 1
        W = tables.shape[1]
        if T > self.max_tokens or S > self.max_seqs or W > self.table_width:
            raise ValueError(f"batch exceeds the runner's limits (T={T}, S={S}, W={W})")
        self.h_tok.numpy()[:T] = toks
        self.h_pos.numpy()[:T] = pos
        self.h_cu.numpy()[:S + 1] = cu
        self.h_tab.numpy()[:S * W] = tables.reshape(-1)
        self.d_tok[:T].copy_(self.h_tok[:T], non_blocking=True)
        self.d_pos[:T].copy_(self.h_pos[:T], non_blocking=True)
        self.d_cu[:S + 1].copy_(self.h_cu[:S + 1], non_blocking=True)
        self.d_tab[:S * W].copy_(self.h_tab[:S * W], non_blocking=True)
        x = self.model.forward(self.cache, self.d_tok[:T], self.d_pos[:T], self.d_cu[:S + 1],
                               self.d_tab[:S * W].view(S, W), self.ws_eager, planned=False)
        R = len(sample_rows)
        if R == 0:
            return self.d_out[:0]
        self.h_rows.numpy()[:R] = sample_rows
        self.d_rows[:R].copy_(self.h_rows[:R], non_blocking=True)
        return self._sample(x.index_select(0, self.d_rows[:R]), temps)

    def run(self, batch, temps: np.ndarray | None = None) -> np.ndarray:
        """One step: decode rows through graphs (chunks of the largest captured size), the rest in
        one eager ragged forward; returns the sampled token per row (-1 where none). temps: per-row
        sampling temperature (None or <= 0: greedy)."""
        S = batch.num_seqs
        out = np.full(S, -1, dtype=np.int64)
        d0, d1 = batch.group_start[0], batch.group_start[1]
        pending = []   # (row indices, device tensor)
        if self.graphs and d1 > d0:
            cap = self.max_graph_batch
            for a in range(d0, d1, cap):
                b = min(d1, a + cap)
                cu = batch.cu_seqlens
                t0 = cu[a:b]
                dev = self._run_graph(batch.tokens[t0], batch.positions[t0], batch.block_tables[a:b],
                                      None if temps is None else temps[a:b])
                self.h_out[:b - a].copy_(dev, non_blocking=False)
                out[a:b] = self.h_out.numpy()[:b - a]
            first_eager = d1
        else:
            first_eager = d0
        if first_eager < S:
            a = first_eager
            cu = batch.cu_seqlens
            t_lo, t_hi = cu[a], cu[S]
            rows_cu = cu[a:] - t_lo
            samp = np.nonzero(batch.samples[a:])[0]
            last_tok = rows_cu[samp + 1] - 1
            tables = batch.block_tables[a:]
            W = min(tables.shape[1], self.table_width)
            dev = self._run_eager(batch.tokens[t_lo:t_hi], batch.positions[t_lo:t_hi], rows_cu, tables[:, :W],
                                  last_tok, None if temps is None else temps[a + samp])
            pending.append((a + samp, dev))
        for idx, dev in pending:
            n = len(idx)
            if n:
                self.h_out[:n].copy_(dev, non_blocking=False)
                out[idx] = self.h_out.numpy()[:n]
        return out
