"""GPU tests of the Qwen3 runner and serving loop on the gfx950 kernels.

The forward pass is checked against a plain PyTorch fp32 restatement of Qwen3 over the same
weights: dense causal attention over K/V quantised per (token, head) to e4m3 exactly as the
cache writer does (scale = max(amax, 1e-8)/448, kernels/fused_ops.cu:127-131,176-180), with the
model's bf16 rounding points (GEMM inputs/outputs, residual stream)."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from cppvllm_amd import ops
from cppvllm_amd.engine_core import Batch
from cppvllm_amd.llm_engine import EngineConfig, LLMEngine, SamplingParams
from cppvllm_amd.runner import Qwen3Config
from tests._util import say

pytestmark = pytest.mark.gpu
DEV = "cuda"
SMALL = Qwen3Config(n_layers=2, vocab_size=4096, max_seq_len=4096)


def _rms(x, w, eps):
    x = x.float()
    return (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)).to(torch.bfloat16).float() * w.float()


def _fp8_fake(x):
    """[T, KV, HD] -> dequantised e4m3 with one scale per (token, head)."""
    sc = x.abs().amax(-1, keepdim=True).clamp_min(1e-8) / 448.0
    q = (x / sc).clamp(-448, 448).to(torch.float8_e4m3fn).float()
    return q * sc


def _linear_bf16(x, w):
    return F.linear(x, w)


def linear_f64(x, w):
    """x . w^T with float64 accumulation, rounded to bf16: the same rounding points as a bf16
    GEMM with another (exact) summation order."""
    return (x.double() @ w.double().T).to(torch.bfloat16)


def ref_forward(m, tokens, positions, linear=_linear_bf16):
    """Plain torch fp32 Qwen3 forward of ONE sequence (all its tokens), returns the final-normed x.
    linear: the bf16 GEMM (torch's by default)."""
    c = m.cfg
    H, KV, HD, eps = c.n_heads, c.n_kv_heads, c.head_dim, c.norm_eps
    T = tokens.numel()
    bf = lambda t: t.to(torch.bfloat16)  # noqa: E731
    h = m.embed[tokens].float()
    cos, sin = m.cos[positions], m.sin[positions]          # [T, HD/2]

    def rope(t):                                            # [T, n, HD] neox
        a, b = t[..., :HD // 2], t[..., HD // 2:]
        cc, ss = cos[:, None, :], sin[:, None, :]
        return torch.cat([a * cc - b * ss, b * cc + a * ss], -1)

    x = _rms(h, m.attn_norm[0], eps)
    mask = torch.ones(T, T, dtype=torch.bool, device=h.device).tril()
    for li in range(c.n_layers):
        qkv = linear(bf(x), m.wqkv[li]).float()
        q = qkv[:, :H * HD].view(T, H, HD)
        k = qkv[:, H * HD:(H + KV) * HD].view(T, KV, HD)
        v = qkv[:, (H + KV) * HD:].view(T, KV, HD)
        q = bf(rope(_rms(q, m.q_norm[li], eps))).float()
        k = bf(rope(_rms(k, m.k_norm[li], eps))).float()
        k, v = _fp8_fake(k), _fp8_fake(v)
        rep = H // KV
        k, v = k.repeat_interleave(rep, 1), v.repeat_interleave(rep, 1)
        s = torch.einsum("thd,shd->hts", q, k) / math.sqrt(HD)
        s = s.masked_fill(~mask, float("-inf"))
        att = torch.einsum("hts,shd->thd", s.softmax(-1), v)
        o = linear(bf(att).reshape(T, H * HD), m.wo[li]).float()
        h = bf(h + o).float()
        x = _rms(h, m.ffn_norm[li], eps)
        gu = linear(bf(x), m.w_gate_up[li]).float()
        g, u = gu[:, :c.intermediate_size], gu[:, c.intermediate_size:]
        act = bf(F.silu(g)).float() * u
        mm = linear(bf(act), m.w_down[li]).float()
        h = bf(h + mm).float()
        nxt = m.attn_norm[li + 1] if li + 1 < c.n_layers else m.final_norm
        x = _rms(h, nxt, eps)
    return x


def _engine(**kw):
    cfg = EngineConfig(block_size=kw.pop("block_size", 16), max_model_len=1024, num_kv_blocks=kw.pop("blocks", 256),
                       max_num_seqs=kw.pop("max_num_seqs", 8), seed=3, weight_std=kw.pop("std", 0.05), **kw)
    return LLMEngine(cfg, SMALL, DEV)


def _batch(lens, positions0, block_size, first_block=0):
    """A ragged batch of len(lens) sequences, sequence j at positions [positions0[j], +lens[j])."""
    toks, pos, cu, tabs = [], [], [0], []
    W = max(-(-(p0 + n) // block_size) for n, p0 in zip(lens, positions0))
    nb = first_block
    for n, p0 in zip(lens, positions0):
        pos.extend(range(p0, p0 + n))
        cu.append(cu[-1] + n)
        k = -(-(p0 + n) // block_size)
        tabs.append(list(range(nb, nb + k)) + [-1] * (W - k))
        nb += k
    T = cu[-1]
    return Batch(tokens=np.zeros(T, np.int64), positions=np.array(pos, np.int64), cu_seqlens=np.array(cu, np.int64),
                 kv_lens=np.array([p + n for n, p in zip(lens, positions0)], np.int64),
                 block_tables=np.array(tabs, np.int64), samples=np.ones(len(lens), bool),
                 seq_ids=np.arange(len(lens), dtype=np.int64), group_start=(0, 0, len(lens), len(lens)))


def test_prefill_and_decode_match_torch_reference():
    say("runner: prefill 3 seqs + graph decode vs torch fp32 reference (2 layers)")
    eng = _engine()
    r, m = eng.runner, eng.model
    g = torch.Generator().manual_seed(21)
    lens = [5, 40, 300]
    b = _batch(lens, [0, 0, 0], 16)
    b.tokens[:] = torch.randint(0, SMALL.vocab_size, (b.num_tokens,), generator=g).numpy()
    # eager prefill: hidden rows of every token
    T, S, W = b.num_tokens, b.num_seqs, b.block_tables.shape[1]
    r._run_eager(b.tokens, b.positions, b.cu_seqlens, b.block_tables, np.array([], np.int64), None)
    x = m.forward(eng.cache, torch.from_numpy(b.tokens).to(DEV), torch.from_numpy(b.positions).to(DEV),
                  torch.from_numpy(b.cu_seqlens).to(DEV), torch.from_numpy(b.block_tables).to(DEV), r.ws_eager,
                  planned=False).float()
    worst = 0.0
    for j in range(S):
        a, e = b.cu_seqlens[j], b.cu_seqlens[j + 1]
        want = ref_forward(m, torch.from_numpy(b.tokens[a:e]).to(DEV), torch.from_numpy(b.positions[a:e]).to(DEV))
        err = (x[a:e] - want).abs()
        say(f"  seq {j} len {e - a}: max-abs {err.max().item():.3e} mean-abs {err.mean().item():.3e}")
        assert err.max().item() < 0.25 and err.mean().item() < 1.5e-2
        worst = max(worst, err.max().item())
    # one decode token per sequence through the captured graph; compare the last row
    new = torch.randint(0, SMALL.vocab_size, (S,), generator=g).numpy()
    d = _batch([1] * S, lens, 16)
    d.tokens[:] = new
    r._stage_graph_rows(d.tokens, d.positions, d.block_tables, 4)
    r.graphs[4].replay()
    torch.cuda.synchronize()
    for j in range(S):
        toks = np.concatenate([b.tokens[b.cu_seqlens[j]:b.cu_seqlens[j + 1]], new[j:j + 1]])
        want = ref_forward(m, torch.from_numpy(toks).to(DEV), torch.arange(len(toks), device=DEV))[-1]
        err = (r.g_hidden[j].float() - want).abs()
        say(f"  decode seq {j}: max-abs {err.max().item():.3e} mean-abs {err.mean().item():.3e}")
        assert err.max().item() < 0.25 and err.mean().item() < 1.5e-2


def test_fused_path_with_norm_gains_matches_torch_reference():
    """Batches of 16..256 rows take the projections with fused epilogues (residual + norm partials,
    row-normed inputs with the gains folded into the weights, QK-norm/RoPE/KV write in the QKV
    epilogue). With random norm gains its rounding points differ from the reference's (the normed
    input is not rounded, the gain-scaled weight is): prefill and decode rows must stay within
    FUSED_X times the error the unfused path (the reference's rounding points, same kernels
    otherwise) shows against the torch fp32 restatement (measured: 1.6-1.8x), and within max-abs
    0.4 / mean-abs 0.04 (random gains widen both paths' errors)."""
    FUSED_X = 2.5
    say("runner: fused-epilogue path with random norm gains vs torch fp32 reference (2 layers)")
    eng = _engine(blocks=128)
    r, m = eng.runner, eng.model
    g = torch.Generator().manual_seed(33)
    gain = lambda n: (torch.rand((n,), generator=g) + 0.5).to(torch.bfloat16).to(DEV)  # noqa: E731
    c = m.cfg
    m.attn_norm = [gain(c.dim) for _ in range(c.n_layers)]
    m.ffn_norm = [gain(c.dim) for _ in range(c.n_layers)]
    m.q_norm = [gain(c.head_dim) for _ in range(c.n_layers)]
    m.k_norm = [gain(c.head_dim) for _ in range(c.n_layers)]
    m.final_norm = gain(c.dim)
    m.fold_gains()
    lens = torch.randint(3, 16, (20,), generator=g).tolist()   # len + 1 <= 16: one block each, both batches
    b = _batch(lens, [0] * 20, 16)
    b.tokens[:] = torch.randint(0, SMALL.vocab_size, (b.num_tokens,), generator=g).numpy()
    new = torch.randint(0, SMALL.vocab_size, (20,), generator=g).numpy()
    dec = _batch([1] * 20, lens, 16)
    dec.tokens[:] = new
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)  # noqa: E731

    def run(bt):
        return m.forward(eng.cache, d(bt.tokens), d(bt.positions), d(bt.cu_seqlens), d(bt.block_tables), r.ws_eager,
                         planned=False).float()

    want_p = torch.cat([ref_forward(m, d(b.tokens[b.cu_seqlens[j]:b.cu_seqlens[j + 1]]),
                                    d(b.positions[b.cu_seqlens[j]:b.cu_seqlens[j + 1]])) for j in range(20)])
    want_d = torch.stack([ref_forward(m, d(np.concatenate([b.tokens[b.cu_seqlens[j]:b.cu_seqlens[j + 1]],
                                                           new[j:j + 1]])),
                                      torch.arange(lens[j] + 1, device=DEV))[-1] for j in range(20)])
    errs = {}
    for fused_path in (False, True):
        m.fused_epilogues = fused_path     # False: the reference's rounding points (EngineConfig.exact_norm_rounding)
        say(f"  {'fused' if fused_path else 'unfused'}: prefill of 20 sequences ({b.num_tokens} rows), "
            "then a 20-row decode step")
        ep = (run(b) - want_p).abs()
        ed = (run(dec) - want_d).abs()
        errs[fused_path] = [(e.max().item(), e.mean().item()) for e in (ep, ed)]
        say(f"    prefill max {errs[fused_path][0][0]:.3e} mean {errs[fused_path][0][1]:.3e}; "
            f"decode max {errs[fused_path][1][0]:.3e} mean {errs[fused_path][1][1]:.3e}")
    m.fold_gains()
    for (fm, fa), (um, ua) in zip(errs[True], errs[False]):
        assert fm < 0.4 and fa < 0.04
        assert fm <= FUSED_X * um and fa <= FUSED_X * ua


def test_graph_decode_equals_eager_decode():
    say("runner: graph replay vs eager forward for the same decode rows")
    eng = _engine()
    r, m = eng.runner, eng.model
    g = torch.Generator().manual_seed(22)
    lens = [17, 64, 3, 100, 250]
    b = _batch(lens, [0] * 5, 16)
    b.tokens[:] = torch.randint(0, SMALL.vocab_size, (b.num_tokens,), generator=g).numpy()
    r._run_eager(b.tokens, b.positions, b.cu_seqlens, b.block_tables, np.array([], np.int64), None)
    d = _batch([1] * 5, lens, 16)
    d.tokens[:] = torch.randint(0, SMALL.vocab_size, (5,), generator=g).numpy()
    cache_k = eng.cache.k.clone()
    r._stage_graph_rows(d.tokens, d.positions, d.block_tables, 8)
    r.graphs[8].replay()
    xg = r.g_hidden[:5].float().clone()
    k_after_graph = eng.cache.k.clone()
    eng.cache.k.copy_(cache_k)
    xe = m.forward(eng.cache, torch.from_numpy(d.tokens).to(DEV), torch.from_numpy(d.positions).to(DEV),
                   torch.from_numpy(d.cu_seqlens).to(DEV), torch.from_numpy(d.block_tables).to(DEV), r.ws_eager,
                   planned=False).float()
    torch.cuda.synchronize()
    # the cache rows written by the decode tokens are identical (same kernel, same inputs) except
    # the scratch block that the idle graph rows wrote
    nb = eng.cache.scratch_block
    assert torch.equal(k_after_graph[:, :nb], eng.cache.k[:, :nb])
    err = (xg - xe).abs()
    assert err.max().item() < 0.1 and err.mean().item() < 5e-3, (err.max().item(), err.mean().item())


@pytest.mark.parametrize("S,B", [(3, 4), (20, 32)])
def test_native_decode_equals_python_forward(S, B):
    """The native decode runner (include/cppvllm_runner.h) and the Python Qwen3.forward over the same
    staged rows (idle rows on the scratch block, planned attention) launch the same kernels with
    the same arguments: hidden rows and cache bytes bit-identical, graph replay and eager forward,
    unfused (B = 4) and fused-epilogue (B = 32) layers."""
    say(f"runner: native decode vs Python forward, {S} rows in a batch of {B}")
    eng = _engine(max_num_seqs=32, blocks=128)
    r, m, cache = eng.runner, eng.model, eng.cache
    g = torch.Generator().manual_seed(27)
    lens = torch.randint(1, 200, (S,), generator=g).tolist()
    b = _batch(lens, [0] * S, 16)
    b.tokens[:] = torch.randint(0, SMALL.vocab_size, (b.num_tokens,), generator=g).numpy()
    r._run_eager(b.tokens, b.positions, b.cu_seqlens, b.block_tables, np.array([], np.int64), None)
    d = _batch([1] * S, lens, 16)
    d.tokens[:] = torch.randint(0, SMALL.vocab_size, (S,), generator=g).numpy()
    snap = [t.clone() for t in (cache.k, cache.v, cache.ks, cache.vs)]
    outs = {}
    for how in ("replay", "eager", "python"):
        for t, s0 in zip((cache.k, cache.v, cache.ks, cache.vs), snap):
            t.copy_(s0)
        if how == "python":
            Wg = r.graph_width
            tab = np.full((B, Wg), -1, np.int64)
            w = min(Wg, d.block_tables.shape[1])
            tab[:S, :w] = d.block_tables[:, :w]
            tab[S:, 0] = cache.scratch_block
            pad = lambda a: np.concatenate([a, np.zeros(B - S, np.int64)])  # noqa: E731
            dv = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)  # noqa: E731
            ws = ops.paged_attention_workspace(B, m.cfg.n_heads, m.cfg.n_kv_heads, m.cfg.head_dim, Wg,
                                               cache.block_size, 0, DEV)
            x = m.forward(cache, dv(pad(d.tokens)), dv(pad(d.positions)), dv(np.arange(B + 1)), dv(tab), ws,
                          planned=True)
        else:
            r._stage_graph_rows(d.tokens, d.positions, d.block_tables, B)
            if how == "replay":
                r.graphs[B].replay()
            else:
                r.decode_eager(B)
            x = r.g_hidden[:B]
        torch.cuda.synchronize()
        outs[how] = (x[:S].clone(), [t.clone() for t in (cache.k, cache.v, cache.ks, cache.vs)])
    for how in ("eager", "python"):
        assert torch.equal(outs[how][0].view(torch.int16), outs["replay"][0].view(torch.int16)), how
        for a, c in zip(outs[how][1], outs["replay"][1]):
            assert torch.equal(a, c), how


def test_eager_engine_equals_graph_engine():
    """enforce_eager runs each decode step through the graph body without capturing it (same
    padding rows, planned attention, partitions and GEMM tilings), so an eager engine and a graph
    engine return the same tokens, including batches that cross graph sizes (1..8 rows)."""
    say("engine: enforce_eager vs HIP graphs, 7 requests, exact tokens")
    g = torch.Generator().manual_seed(26)
    prompts = [torch.randint(0, SMALL.vocab_size, (n,), generator=g).tolist() for n in (5, 70, 33, 140, 9, 18, 2)]
    params = [SamplingParams(max_tokens=n, ignore_eos=True) for n in (20, 3, 17, 9, 25, 40, 11)]
    outs = [_engine(enforce_eager=eager, max_num_seqs=8, blocks=96).generate(prompts, params)
            for eager in (True, False)]
    assert outs[0] == outs[1]
    assert [len(o) for o in outs[0]] == [20, 3, 17, 9, 25, 40, 11]


def test_generate_greedy_with_chunked_prefill_and_graphs():
    say("engine: generate 6 requests, chunked prefill (64-token budget), graphs on")
    eng = _engine(max_num_batched_tokens=64, max_chunk_tokens=32, max_num_seqs=4, blocks=64)
    g = torch.Generator().manual_seed(23)
    prompts = [torch.randint(0, SMALL.vocab_size, (n,), generator=g).tolist() for n in (3, 50, 130, 7, 64, 20)]
    outs = eng.generate(prompts, [SamplingParams(max_tokens=n, ignore_eos=True) for n in (5, 9, 3, 12, 1, 30)])
    assert [len(o) for o in outs] == [5, 9, 3, 12, 1, 30]
    assert all(0 <= t < SMALL.vocab_size for o in outs for t in o)
    st = eng.stats()
    assert st.tokens_sampled == 60 and st.finished == 6
    # the same requests alone, eagerly: the first generated token (prefill logits) agrees
    eng2 = _engine(enforce_eager=True, max_num_seqs=4, blocks=64, depth=1)
    first = [eng2.generate([p], SamplingParams(max_tokens=1, ignore_eos=True))[0][0] for p in prompts]
    agree = sum(int(a[0] == b) for a, b in zip(outs, first))
    assert agree >= 5, (outs, first)


def test_launch_ring_equals_synchronous_steps():
    say("engine: two-deep launch ring (device token feedback) vs synchronous steps")
    g = torch.Generator().manual_seed(24)
    prompts = [torch.randint(0, SMALL.vocab_size, (n,), generator=g).tolist() for n in (5, 70, 33, 140, 9)]
    params = [SamplingParams(max_tokens=n, ignore_eos=True) for n in (20, 3, 17, 9, 25)]
    outs = []
    for depth in (1, 2):
        eng = _engine(depth=depth, max_num_seqs=8, blocks=64)
        outs.append(eng.generate(prompts, params))
        assert eng.core.outstanding() == 0 and eng.stats().free_blocks == 64
    assert outs[0] == outs[1]
    assert [len(o) for o in outs[1]] == [20, 3, 17, 9, 25]


@pytest.mark.parametrize("B", [4, 16])
def test_shared_prefix_decode_matches_torch_reference(B):
    """Decode rows whose tables share their first 4 blocks (a 64-token common prefix), through the
    shared-prefix graph (the plan groups them into one unit that reads the prefix once) and the
    plain graph: both within the bar of the fp32 restatement, and close to each other."""
    say(f"runner: shared-prefix decode graph (units) vs plain graph vs torch reference, batch {B}")
    eng = _engine(max_num_seqs=16, blocks=128)
    r, m = eng.runner, eng.model
    g = torch.Generator().manual_seed(28)
    common = torch.randint(0, SMALL.vocab_size, (64,), generator=g).numpy()
    lens = [64 + n for n in (3, 10, 21)] + [40]          # three sharers and one other sequence
    prompts = [np.concatenate([common, torch.randint(0, SMALL.vocab_size, (n - 64,), generator=g).numpy()])
               for n in lens[:3]] + [torch.randint(0, SMALL.vocab_size, (lens[3],), generator=g).numpy()]
    W = 6
    tab = np.full((4, W), -1, np.int64)
    nxt = 4
    for i, n in enumerate(lens):
        k = -(-(n + 1) // 16)
        row = list(range(4)) + list(range(nxt, nxt + k - 4)) if i < 3 else list(range(nxt, nxt + k))
        nxt += len(row) - (4 if i < 3 else 0)
        tab[i, :k] = row
    shared = np.array([4, 4, 4, 0], np.int32)
    # prefill: the sharers' common blocks are written by the first sequence only (prefix-cache hit)
    toks = np.concatenate([prompts[0], *(p[64:] for p in prompts[1:3]), prompts[3]])
    pos = np.concatenate([np.arange(lens[0]), *(np.arange(64, n) for n in lens[1:3]), np.arange(lens[3])])
    cu = np.cumsum([0, lens[0], lens[1] - 64, lens[2] - 64, lens[3]])
    r._run_eager(toks, pos, cu, tab, np.array([], np.int64), None)
    new = torch.randint(0, SMALL.vocab_size, (4,), generator=g).numpy()
    dpos = np.asarray(lens, np.int64)
    outs = {}
    snap = [t.clone() for t in (eng.cache.k, eng.cache.v, eng.cache.ks, eng.cache.vs)]
    for use_shared in (True, False):
        for t, s0 in zip((eng.cache.k, eng.cache.v, eng.cache.ks, eng.cache.vs), snap):
            t.copy_(s0)
        r._stage_graph_rows(new, dpos, tab, B, shared=shared if use_shared else None)
        (r.graphs_shared if use_shared else r.graphs)[B].replay()
        torch.cuda.synchronize()
        outs[use_shared] = r.g_hidden[:4].float().clone()
    for j in range(4):
        seq = torch.from_numpy(np.concatenate([prompts[j], new[j:j + 1]])).to(DEV)
        want = ref_forward(m, seq, torch.arange(seq.numel(), device=DEV))[-1]
        for use_shared in (True, False):
            err = (outs[use_shared][j] - want).abs()
            say(f"  seq {j} shared={use_shared}: max-abs {err.max().item():.3e} mean-abs {err.mean().item():.3e}")
            assert err.max().item() < 0.25 and err.mean().item() < 1.5e-2
    d = (outs[True] - outs[False]).abs()
    say(f"  shared vs plain: max-abs {d.max().item():.3e} mean-abs {d.mean().item():.3e}")
    assert d.max().item() < 0.1 and d.mean().item() < 5e-3


def test_prefix_cache_sharing_uses_shared_graphs():
    """Requests that hit the prefix cache decode through the shared-prefix graphs (units that read
    the common blocks once). Their numerics are checked against the fp32 restatement in
    test_shared_prefix_decode_matches_torch_reference; here the engine runs both ways, returns every
    token count, and agrees on the first token (from the prefill, which units do not touch). Later
    tokens may differ where two logits tie within the rounding of another summation order."""
    say("engine: prefix-cache hits -> decode graphs with shared-prefix units")
    g = torch.Generator().manual_seed(25)
    common = torch.randint(0, SMALL.vocab_size, (64,), generator=g).tolist()       # 4 full 16-token blocks
    prompts = [common + torch.randint(0, SMALL.vocab_size, (n,), generator=g).tolist() for n in (3, 10, 21, 5)]
    params = SamplingParams(max_tokens=12, ignore_eos=True)
    outs = []
    for use_shared in (True, False):
        eng = _engine(max_num_seqs=8, blocks=64)
        if not use_shared:
            eng.runner.graphs_shared = eng.runner.graphs
        first = eng.generate(prompts[:1], params)          # fills the prefix cache
        rest = eng.generate(prompts[1:], params)           # three requests hit the 4 common blocks
        outs.append(first + rest)
        assert eng.stats().prefix_hit_tokens >= 3 * 64
        assert [len(o) for o in outs[-1]] == [12] * 4
        if use_shared:
            assert eng.runner.shared_replays > 0
    assert outs[0][0] == outs[1][0]
    assert [o[0] for o in outs[0]] == [o[0] for o in outs[1]]

def _teacher_forced_gaps(m, prompt, out):
    """Run prompt + out through the torch fp32 restatement (ref_forward) in one pass and return,
    for every generated token, how far its logit lies below that position's largest logit."""
    toks = torch.tensor(prompt + out, device=DEV)
    x = ref_forward(m, toks, torch.arange(len(toks), device=DEV))
    lg = x[len(prompt) - 1:len(prompt) - 1 + len(out)].to(torch.bfloat16).float() @ m.embed.float().T
    chosen = lg[torch.arange(len(out), device=DEV), torch.tensor(out, device=DEV)]
    return lg.max(-1).values - chosen


def test_preemption_by_recompute_keeps_outputs():
    """A 16-block pool (256 cache slots) for six requests that need ~650: running sequences are
    preempted when blocks run out (engine/scheduler.cpp: the newest running sequence is evicted and
    later recomputed as a prefill of its whole context). Every request still produces its token
    count and the pool is whole again at the end.
    Tokens: every generated token of both this run and a run whose pool never fills is checked by
    teacher forcing against the torch fp32 restatement (the prompt plus the run's own tokens in one
    pass): each must lie within GAP logits of the restatement's largest logit at its position, and at
    most 10% may differ from that argmax. The weights (N(0, 0.5)) give logits with a standard
    deviation of ~16 (top-1/top-2 margins ~3 at the median), the engine's bf16 roundings move them by
    well under 1, while a recompute that wrote wrong K/V (positions, slots, scales) would pick tokens
    tens of logits below the maximum. The two runs need not agree token for token: their batches
    differ after the preemption (other row counts pick other GEMM tilings and attention partitions,
    so bf16 roundings differ), so where they first diverge both tokens must be near-ties there."""
    GAP = 2.0
    say("engine: preemption by recompute with a 16-block pool")
    g = torch.Generator().manual_seed(31)
    lens, outs_n = (40, 70, 33, 90, 25, 60), (60, 40, 80, 30, 70, 50)
    prompts = [torch.randint(0, SMALL.vocab_size, (n,), generator=g).tolist() for n in lens]
    params = [SamplingParams(max_tokens=n, ignore_eos=True) for n in outs_n]
    small = _engine(max_num_seqs=6, blocks=16, std=0.5)
    got = small.generate(prompts, params)
    st = small.stats()
    assert st.preemptions >= 1 and st.free_blocks == 16
    assert [len(o) for o in got] == list(outs_n)
    big = _engine(max_num_seqs=6, blocks=256, std=0.5)
    want = big.generate(prompts, params)
    assert big.stats().preemptions == 0
    m = small.model
    for i, (p, a, b) in enumerate(zip(prompts, got, want)):
        for name, out in (("preempted", a), ("unpreempted", b)):
            gap = _teacher_forced_gaps(m, p, out)
            off = int((gap > 0).sum())
            say(f"  request {i} {name}: max gap {gap.max().item():.3f}, {off} of {len(out)} off the argmax")
            assert gap.max().item() <= GAP and off <= len(out) // 10
        d = next((k for k in range(len(a)) if a[k] != b[k]), None)
        if d is not None:                  # a near-tie under the restatement where the runs part
            gap = _teacher_forced_gaps(m, p + a[:d], [a[d]]).item(), _teacher_forced_gaps(m, p + a[:d], [b[d]]).item()
            say(f"  request {i}: runs part at token {d}, gaps {gap[0]:.3f} / {gap[1]:.3f}")
            assert max(gap) <= GAP


def test_runner_stage_rejects_positions_past_the_table():
    """cvh_runner_stage accepts the last position the runner's table width covers and rejects one
    past it (the kernels would clamp the context instead of attending it) and a negative one."""
    from cppvllm_amd import _lib
    say("native runner: staged positions checked against the table width")
    eng = _engine(blocks=64)
    r = eng.runner
    W, BS = r.graph_width, eng.cfg.block_size
    t = np.zeros(1, np.int64)
    tab = np.zeros((1, W), np.int64)
    stream = torch.cuda.current_stream().cuda_stream
    for pos, want in ((W * BS - 1, 0), (W * BS, _lib.CVH_ERR_INVALID_ARG), (-1, _lib.CVH_ERR_INVALID_ARG)):
        p = np.array([pos], np.int64)
        rc = r._L.cvh_runner_stage(r._handle, 0, 1, 1, t.ctypes.data, p.ctypes.data, tab.ctypes.data, W, None, None,
                                   None, stream)
        assert rc == want, (pos, rc)
    torch.cuda.synchronize()
