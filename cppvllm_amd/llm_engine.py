"""Request-level engine: the serving loop around the native scheduler and the model runner.

Mirrors LLMEngine (engine/llm_engine.h:34-69, engine/llm_engine.cpp:30-155): ``add_request``,
``step`` (a two-deep ring of schedule -> launch, then collect -> postprocess), ``is_finished``,
``generate``, ``stats``. Scheduling
and the paged block manager are the C++ core (include/cppvllm_engine.h); the step runs on the
gfx950 kernels through ``ModelRunner``.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from .engine_core import EngineBusy, EngineCore
from .runner import KVCache, ModelRunner, Qwen3, Qwen3Config


@dataclass
class SamplingParams:
    """sequence.h:20-24 (temperature <= 0 is greedy)."""
    temperature: float = 0.0
    max_tokens: int = 64
    ignore_eos: bool = False


@dataclass
class EngineConfig:
    """config.h:62-79, plus the KV block size (16 in the reference, a runtime power of two here)."""
    max_num_batched_tokens: int = 4096
    max_num_seqs: int = 256
    max_chunk_tokens: int = 1024
    max_model_len: int = 4096
    block_size: int = 256
    gpu_memory_utilization: float = 0.90
    num_kv_blocks: int = -1
    enforce_eager: bool = False
    depth: int = 2                 # outstanding steps (llm_engine.h:51 kDepth); 1 = synchronous
    seed: int = 0
    weight_std: float = 0.02
    eos_token_id: int = 151645
    # True: every step rounds at the reference's points (add_rms_norm output rounded to bf16 before
    # each projection); False: decode batches of 16-256 rows use the fused-epilogue projections
    exact_norm_rounding: bool = False
    extra: dict = field(default_factory=dict)


class LLMEngine:
    def __init__(self, cfg: EngineConfig | None = None, model_cfg: Qwen3Config | None = None, device="cuda"):
        self.cfg = cfg = cfg or EngineConfig()
        self.model_cfg = mc = model_cfg or Qwen3Config()
        self.device = torch.device(device)
        self.model = Qwen3(mc, self.device, seed=cfg.seed, std=cfg.weight_std)
        self.model.fused_epilogues = not cfg.exact_norm_rounding
        self.num_blocks = self._size_kv_cache()
        self.cache = KVCache(mc, self.num_blocks, cfg.block_size, self.device)
        self.runner = ModelRunner(self.model, self.cache, max_num_batched_tokens=cfg.max_num_batched_tokens,
                                  max_num_seqs=cfg.max_num_seqs, max_model_len=cfg.max_model_len,
                                  enforce_eager=cfg.enforce_eager, seed=cfg.seed)
        self.core = EngineCore(max_num_batched_tokens=cfg.max_num_batched_tokens, max_num_seqs=cfg.max_num_seqs,
                               max_chunk_tokens=cfg.max_chunk_tokens, block_size=cfg.block_size,
                               num_blocks=self.num_blocks, graph_max_blocks=self.runner.graph_width,
                               eos_token_id=cfg.eos_token_id)
        self.temps: dict[int, float] = {}
        self._ring: list = []             # (batch, runner handle) of launched, unprocessed steps

    def _size_kv_cache(self) -> int:
        """Blocks that fit in gpu_memory_utilization of the device after the weights
        (model_runner.cpp:116-145), capped at what max_num_seqs full-length sequences can use."""
        cfg, mc = self.cfg, self.model_cfg
        per_block = KVCache.bytes_per_block(mc, cfg.block_size)
        want = cfg.max_num_seqs * -(-cfg.max_model_len // cfg.block_size)
        if cfg.num_kv_blocks > 0:
            return cfg.num_kv_blocks
        free, total = torch.cuda.mem_get_info(self.device)
        budget = int(free - (1.0 - cfg.gpu_memory_utilization) * total) - (4 << 30)   # activations, graphs
        n = min(want, budget // per_block)
        if n <= 0:
            raise RuntimeError("no device memory left for the KV cache")
        return n

    def add_request(self, prompt, params: SamplingParams | None = None) -> int:
        p = params or SamplingParams()
        rid = self.core.add_request(prompt, p.max_tokens, p.ignore_eos)
        if p.temperature > 0:
            self.temps[rid] = float(p.temperature)
        return rid

    def step(self) -> int:
        """Advance the two-deep launch ring (engine/llm_engine.cpp:70-113): schedule and launch
        the next step when fewer than two are outstanding, and post-process the oldest one once two
        are (or when nothing else can be scheduled). Returns the number of tokens sampled by the
        step post-processed in this call (0 if none was)."""
        if len(self._ring) < self.cfg.depth:
            try:
                batch = self.core.schedule()
            except EngineBusy:
                batch = None
            if batch is not None:
                temps = None
                if self.temps:
                    temps = np.array([self.temps.get(int(r), 0.0) for r in batch.seq_ids], dtype=np.float32)
                self._ring.append((batch, self.runner.launch(batch, temps)))
                if len(self._ring) < self.cfg.depth:
                    return 0
        if not self._ring:
            return 0
        batch, handle = self._ring.pop(0)
        self.core.postprocess(self.runner.collect(handle))
        return int(np.count_nonzero(batch.samples))

    def is_finished(self) -> bool:
        return self.core.is_finished()

    def take_finished(self) -> dict[int, list[int]]:
        out = self.core.take_finished()
        for rid in out:
            self.temps.pop(rid, None)
        return out

    def generate(self, prompts, params) -> list[list[int]]:
        """Run prompts to completion; returns the generated tokens of each prompt, in order."""
        if isinstance(params, SamplingParams):
            params = [params] * len(prompts)
        ids = [self.add_request(p, sp) for p, sp in zip(prompts, params)]
        done: dict[int, list[int]] = {}
        while not self.is_finished():
            self.step()
            done.update(self.take_finished())
        done.update(self.take_finished())
        return [done[i] for i in ids]

    def stats(self):
        return self.core.stats()
