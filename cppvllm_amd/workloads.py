"""Seeded synthetic ragged batches for the hot path (host side of the runner).

Each builder returns a dict of torch tensors on ``device``. Small metadata (lengths, block
permutations) comes from a CPU generator seeded with ``seed`` so it is identical on every
machine; bulk K/V/q data comes from a generator on ``device``.

Layouts follow the reference runner (engine/model_runner.cpp:104-113, :296-308):
  k_cache/v_cache uint8 [NB, BS, KV, HD]; scales float32 with memory order [NB][KV][BS]
  (exposed as a [NB, BS, KV]-shaped view is not needed here, so they are stored [NB, KV, BS]);
  block_tables int64 [S, W] padded with -1.

Shapes: Qwen3-0.6B attention (config.h:13-25): 16 query heads, 8 kv heads, head_dim 128.
"""
from __future__ import annotations

import math

import torch

H, KV, HD = 16, 8, 128
HIDDEN = 1024
E4M3_MAX = 448.0


def _cpu_gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _dev_gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def quantize_blocks(x: torch.Tensor, per_tensor: bool, tensor_scale: float | None = None):
    """x float [NB, BS, KV, HD] -> (codes uint8 [NB, BS, KV, HD], scales).

    Per-(token, head): scale = max(amax, 1e-8)/448 stored [NB, KV, BS] (fused_ops.cu:127-136).
    Per-tensor: one float32 scale (absmax/448 unless given).
    """
    if per_tensor:
        sc = float(x.abs().max()) / E4M3_MAX if tensor_scale is None else tensor_scale
        codes = (x / sc).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn).view(torch.uint8)
        return codes, torch.tensor([sc], dtype=torch.float32, device=x.device)
    amax = x.abs().amax(dim=-1, keepdim=True).clamp_min(1e-8)
    sc = amax / E4M3_MAX
    codes = (x / sc).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn).view(torch.uint8)
    return codes, sc.squeeze(-1).permute(0, 2, 1).contiguous().float()


def _fill_cache(nb: int, bs: int, per_tensor: bool, gen: torch.Generator, device, outlier_frac: float = 0.0,
                chunk_blocks: int = 256):
    """Random N(0,1) K or V for every slot of an nb-block pool, quantised to e4m3."""
    codes = torch.empty((nb, bs, KV, HD), dtype=torch.uint8, device=device)
    scales = torch.empty((nb, KV, bs), dtype=torch.float32, device=device)
    xs = []
    for b0 in range(0, nb, chunk_blocks):
        b1 = min(nb, b0 + chunk_blocks)
        x = torch.randn((b1 - b0, bs, KV, HD), generator=gen, device=device, dtype=torch.float32)
        if outlier_frac > 0:
            mask = torch.rand(x.shape, generator=gen, device=device) < outlier_frac
            x = torch.where(mask, x * 20.0, x)
        if per_tensor:
            xs.append(x)
        else:
            c, s = quantize_blocks(x, False)
            codes[b0:b1] = c
            scales[b0:b1] = s
    if per_tensor:
        amax = max(float(x.abs().max()) for x in xs)
        sc = amax / E4M3_MAX
        b0 = 0
        for x in xs:
            c, _ = quantize_blocks(x, True, sc)
            codes[b0:b0 + x.shape[0]] = c
            b0 += x.shape[0]
        scales = torch.tensor([sc], dtype=torch.float32, device=device)
    return codes, scales


def decode_batch(ctx_lens: list[int], bs: int, seed: int, device="cpu", per_tensor: bool = False,
                 pool_blocks: int | None = None, outlier_frac: float = 0.0, shared_prefix_blocks: int = 0):
    """One decode step: one query token per sequence at position ctx-1 (kv_len = ctx).

    Physical blocks are a seeded random permutation of the pool, handed out sequence by sequence
    (the block manager's free-list order is an arbitrary permutation too). With
    shared_prefix_blocks = n, every even sequence's first n table entries are the same physical
    blocks (a prefix-cache hit, engine/block_manager.cpp:80-116).
    """
    g = _cpu_gen(seed)
    S = len(ctx_lens)
    nblk = [math.ceil(c / bs) for c in ctx_lens]
    need = sum(nblk)
    if shared_prefix_blocks:
        need -= sum(min(shared_prefix_blocks, n) for i, n in enumerate(nblk) if i % 2 == 0 and i > 0)
    nb = max(need, pool_blocks or 0)
    perm = torch.randperm(nb, generator=g).tolist()
    W = max(nblk)
    table = torch.full((S, W), -1, dtype=torch.int64)
    it = iter(perm)
    shared = None
    for i, n in enumerate(nblk):
        row = []
        for b in range(n):
            if shared_prefix_blocks and i % 2 == 0 and shared is not None and b < min(shared_prefix_blocks, len(shared)):
                row.append(shared[b])
            else:
                row.append(next(it))
        if shared_prefix_blocks and i == 0:
            shared = row[:shared_prefix_blocks]
        table[i, :n] = torch.tensor(row, dtype=torch.int64)
    dg = _dev_gen(seed + 1, device)
    k_cache, k_scale = _fill_cache(nb, bs, per_tensor, dg, device, outlier_frac)
    v_cache, v_scale = _fill_cache(nb, bs, per_tensor, dg, device, outlier_frac)
    q = torch.randn((S, H, HD), generator=dg, device=device, dtype=torch.float32).to(torch.bfloat16)
    return {
        "q": q,
        "k_cache": k_cache, "v_cache": v_cache, "k_scale": k_scale, "v_scale": v_scale,
        "block_tables": table.to(device),
        "token_seq": torch.arange(S, dtype=torch.int64).to(device),
        "token_kv_len": torch.tensor(ctx_lens, dtype=torch.int64).to(device),
        "block_size": bs, "n_heads": H, "n_kv_heads": KV, "head_dim": HD,
        "scale": 1.0 / math.sqrt(HD), "num_blocks": nb,
        # leading blocks of each table row that other rows also reference (prefix-cache hits)
        "shared_blocks": torch.tensor([min(shared_prefix_blocks, n) if (shared_prefix_blocks and i % 2 == 0) else 0
                                       for i, n in enumerate(nblk)], dtype=torch.int32).to(device),
    }


def tp_share(b: dict, tp: int) -> dict:
    """The first GPU's shard of a decode batch under tensor parallelism over kv heads (the
    reference's scaffold divides n_heads and n_kv_heads by tp, model_architecture.cpp:59-62):
    kv heads [0, KV/tp) of the caches and scales and their query heads [0, H/tp); tables,
    contexts and block pool unchanged."""
    kv, h = b["n_kv_heads"] // tp, b["n_heads"] // tp
    out = dict(b)
    out["k_cache"] = b["k_cache"][:, :, :kv].contiguous()
    out["v_cache"] = b["v_cache"][:, :, :kv].contiguous()
    if b["k_scale"].dim() == 3:
        out["k_scale"] = b["k_scale"][:, :kv].contiguous()
        out["v_scale"] = b["v_scale"][:, :kv].contiguous()
    out["q"] = b["q"][:, :h].contiguous()
    out["n_kv_heads"], out["n_heads"] = kv, h
    return out


def config1_lens(seed: int = 1001, S: int = 8) -> list[int]:
    g = _cpu_gen(seed)
    return torch.randint(100, 1025, (S,), generator=g).tolist()


def config1(device="cpu", per_tensor=True, seed=1001):
    """8 sequences, ctx ~ U{100..1024}, 256-token blocks from a 64-block pool."""
    return decode_batch(config1_lens(seed), 256, seed, device, per_tensor, pool_blocks=64)


def config3_lens(seed: int = 1003, S: int = 256) -> list[int]:
    g = _cpu_gen(seed)
    a = torch.randint(100, 1025, (S,), generator=g)
    b = torch.randint(0, 1025, (S,), generator=g)
    return (a + b).tolist()


def config3(device="cpu", per_tensor=False, seed=1003, seqs: int = 256):
    """Headline: 256 sequences, ctx = U{100..1024} + U{0..1024}, 256-token blocks (`seqs` other
    than 256: the same distribution over fewer or more sequences, a smaller decode batch)."""
    return decode_batch(config3_lens(seed, seqs), 256, seed, device, per_tensor)


def config4_lens(seed: int = 1004, S: int = 64, lo: int = 4096, hi: int = 32768) -> list[int]:
    g = _cpu_gen(seed)
    u = torch.rand((S,), generator=g, dtype=torch.float64)
    return [int(round(math.exp(math.log(lo) + float(x) * (math.log(hi) - math.log(lo))))) for x in u]


def config4(device="cpu", per_tensor=False, seed=1004, shared_prefix=False):
    """Split-K: 64 sequences, ctx log-uniform in [4k, 32k], 1% outliers at 20x; optional
    shared 8-block prefix on every even sequence."""
    return decode_batch(config4_lens(seed), 256, seed, device, per_tensor, outlier_frac=0.01,
                        shared_prefix_blocks=8 if shared_prefix else 0)


def prefill_lens(seed: int = 1005, T: int = 4096) -> list[int]:
    """Prompt lengths U{100..1024} (config 5's inputs) filling one T-token prefill step; the last
    prompt is cut so that the lengths sum to T (the engine's token budget, scheduler.cpp:60-80)."""
    g = _cpu_gen(seed)
    lens = []
    while sum(lens) < T:
        lens.append(int(torch.randint(100, 1025, (1,), generator=g)))
    lens[-1] -= sum(lens) - T
    return lens


def prefill_batch(lens: list[int], bs: int, seed: int, device="cpu"):
    """One fresh-prefill step: every position of every prompt is a query token (causal
    kv_len = pos + 1), K/V of the whole prompts already in the cache."""
    b = decode_batch(lens, bs, seed, device)
    tseq, tlen = [], []
    for i, L in enumerate(lens):
        tseq += [i] * L
        tlen += list(range(1, L + 1))
    T = len(tseq)
    dg = _dev_gen(seed + 2, device)
    b["q"] = torch.randn((T, H, HD), generator=dg, device=device, dtype=torch.float32).to(torch.bfloat16)
    b["token_seq"] = torch.tensor(tseq, dtype=torch.int64).to(device)
    b["token_kv_len"] = torch.tensor(tlen, dtype=torch.int64).to(device)
    return b


def attention_flops(kv_lens, n_heads=H, hd=HD) -> int:
    """q.k and p.v multiply-adds of every (query token, head, key): 4*hd flop per key and head."""
    return int(sum(kv_lens)) * n_heads * hd * 4


def attention_bytes(kv_lens, n_kv=KV, hd=HD, n_heads=H, per_tensor=False) -> int:
    """Algorithmic HBM bytes of one paged-attention call: every context key's K and V row of each
    kv head (+ 8 B of scales per (key, head) in per-token mode), plus q in and out (bf16)."""
    tokens = int(sum(int(x) for x in kv_lens))
    per_key = n_kv * (2 * hd + (0 if per_tensor else 8))
    return tokens * per_key + 2 * len(kv_lens) * n_heads * hd * 2


def fused_batch(seed: int = 1002, device="cpu", T: int = 4096, n_segments: int = 32, bs: int = 256,
                per_tensor: bool = False, pad_rows: int = 64):
    """Config 2: packed ragged batch of T tokens for add_rms_norm and qk_norm_rope_kv_write.

    Segments (lengths U{16..256}, positions continuing a cached prefix of U{0..1024} tokens) fill
    at most T - pad_rows rows (the last segment is truncated); the remaining rows are padding with
    slot -1 and position 0, like the idle rows of a captured decode batch."""
    g = _cpu_gen(seed)
    lens = torch.randint(16, 257, (n_segments,), generator=g).tolist()
    offs = torch.randint(0, 1025, (n_segments,), generator=g).tolist()
    total = 0
    seg = []
    for L, o in zip(lens, offs):
        L = min(L, T - pad_rows - total)
        if L <= 0:
            break
        seg.append((L, o))
        total += L
    positions = torch.zeros(T, dtype=torch.int64)
    slots = torch.full((T,), -1, dtype=torch.int64)
    nblk = [math.ceil((o + L) / bs) for L, o in seg]
    nb = sum(nblk) + 1
    perm = torch.randperm(nb, generator=g).tolist()
    t = 0
    p = 0
    for (L, o), n in zip(seg, nblk):
        table = perm[p:p + n]
        p += n
        for k in range(L):
            pos = o + k
            positions[t] = pos
            slots[t] = table[pos // bs] * bs + pos % bs
            t += 1
    dg = _dev_gen(seed + 1, device)
    n_tasks = H + 2 * KV

    def bf(shape):
        return torch.randn(shape, generator=dg, device=device, dtype=torch.float32).to(torch.bfloat16)

    def gamma(n):
        return (torch.rand((n,), generator=dg, device=device) + 0.5).to(torch.bfloat16)

    return {
        "resid": bf((T, HIDDEN)), "x": bf((T, HIDDEN)), "w": gamma(HIDDEN),
        "qkv": bf((T, n_tasks * HD)), "q_norm": gamma(HD), "k_norm": gamma(HD),
        "positions": positions.to(device), "slots": slots.to(device), "num_blocks": nb, "block_size": bs,
        "valid_tokens": total, "n_heads": H, "n_kv_heads": KV, "head_dim": HD, "eps": 1e-6, "theta": 1e6,
        "max_position": max(o + L for L, o in seg) + 1,
    }
