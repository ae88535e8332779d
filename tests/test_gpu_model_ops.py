"""GPU parity of the model ops around the attention path (SwiGLU, sampler, token feedback,
embedding) against the CPU oracle, through the C ABI."""
import numpy as np
import pytest
import torch

from cppvllm_amd import ops
from tests._util import np_, say

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("T,I,dtype", [(256, 3072, torch.bfloat16), (7, 100, torch.bfloat16),
                                       (33, 3072, torch.float16), (9, 64, torch.float32), (1, 8, torch.bfloat16)])
def test_swiglu_bitexact(orc, T, I, dtype):
    say(f"swiglu T={T} I={I} {dtype}")
    g = torch.Generator().manual_seed(T * 7 + I)
    gu = (torch.randn((T, 2 * I), generator=g) * 3).to(dtype)
    gu[0, :4] = torch.tensor([0.0, 40.0, -40.0, 1e-3]).to(dtype)
    out = torch.empty((T, I), dtype=dtype, device=DEV)
    ops.fused.swiglu(out, gu.to(DEV))
    torch.cuda.synchronize()
    dt = {torch.bfloat16: orc.BF16, torch.float16: orc.F16, torch.float32: orc.F32}[dtype]
    src = np_(gu) if dtype != torch.float16 else gu.view(torch.int16).numpy().view(np.uint16)
    want = orc.swiglu(src, dtype=dt)
    got = np_(out) if dtype != torch.float16 else out.cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


def test_swiglu_every_bf16_gate(orc):
    """Every one of the 65536 bf16 gate values (NaN, infinities, subnormals included) gives the
    oracle's result bit for bit, with u = 1 (silu itself) and with random u."""
    say("swiglu over every bf16 gate value")
    g_bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).reshape(64, 1024)
    gen = torch.Generator().manual_seed(17)
    for u in (torch.ones((64, 1024)).to(torch.bfloat16), (torch.randn((64, 1024), generator=gen) * 3).to(torch.bfloat16)):
        gu = torch.cat([g_bits, u], dim=1)
        out = torch.empty((64, 1024), dtype=torch.bfloat16, device=DEV)
        ops.fused.swiglu(out, gu.to(DEV))
        torch.cuda.synchronize()
        want = orc.swiglu(np_(gu), dtype=orc.BF16)
        got = np_(out)
        bad = np.nonzero(got != want)
        assert bad[0].size == 0, f"{bad[0].size} mismatches, first at {bad[0][0]},{bad[1][0]}"


@pytest.mark.parametrize("ldtype", [torch.float32, torch.bfloat16])
def test_greedy_sampler_full_vocab(orc, ldtype):
    say(f"greedy sampler R=256 V=151936 {ldtype}")
    g = torch.Generator().manual_seed(11)
    R, V = 256, 151936
    lg = torch.randn((R, V), generator=g).to(ldtype)
    lg[3, [17, 90000, 151935]] = 40.0            # ties -> lowest index
    lg[4, -1] = 60.0                              # max in the last element
    lg[5, 0] = 60.0
    lg[6, :] = float("-inf")
    lg[7, 5] = float("nan")
    lg[8, :] = float("nan")                       # nothing wins: the (-inf, 0x7FFFFFFF) start stays
    lg[9, :] = float("nan")
    lg[9, 70000] = float("-inf")                  # -inf beats NaN
    lg[10, :] = 1.0                               # all equal: index 0
    lg[11, :] = -1.0
    lg[11, 300], lg[11, 9000] = -0.0, 0.0         # signed zeros tie: the lower index (-0.0) wins
    lg[12, :] = -1.0
    lg[12, 300], lg[12, 9000] = 0.0, -0.0
    out = torch.empty(R, dtype=torch.int64, device=DEV)
    ops.fused.sample_tokens(out, lg.to(DEV), None, None, 0, 0)
    torch.cuda.synchronize()
    want = orc.sample_tokens(np_(lg))
    got = out.cpu().numpy()
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"rows {bad[:8]}: got {got[bad[:8]]} want {want[bad[:8]]}"
    assert want[3] == 17 and want[4] == V - 1 and want[5] == 0 and want[6] == 0
    assert want[8] == 0x7FFFFFFF and want[9] == 70000 and want[10] == 0
    assert want[11] == 300 and want[12] == 300
    assert torch.signbit(lg[11, 300]) and not torch.signbit(lg[11, 9000])


def test_sampler_rows_and_temperatures(orc):
    say("gumbel sampler rows/temps R=8 V=151936, 1003, 8, 7, 1")
    g = torch.Generator().manual_seed(12)
    for V in (151936, 1003, 8, 7, 1):
        lg = torch.randn((10, V), generator=g)
        rows = torch.tensor([9, 0, 3, 3, 5, 1, 2, 8], dtype=torch.int64)
        temps = torch.tensor([0.6, 1.0, 0.0, 0.6, 2.0, -1.0, 1e-6, 0.3], dtype=torch.float32)
        out = torch.empty(8, dtype=torch.int64, device=DEV)
        seed, off = 0xDEADBEEF12345678, 3
        ops.fused.sample_tokens(out, lg.to(DEV), rows.to(DEV), temps.to(DEV), seed, off)
        torch.cuda.synchronize()
        want = orc.sample_tokens(lg.numpy(), rows=rows.numpy(), temps=temps.numpy(), seed=seed, offset=off)
        got = out.cpu().numpy()
        assert np.array_equal(got, want), f"V={V}: got {got} want {want}"


def test_sampler_extreme_temperatures_and_logits(orc):
    """Gumbel rows at temperatures 1e-30 (x / t overflows to +-inf), 1e30 (the noise decides) and
    1, on logits with +-inf, NaN and 1e38 entries, against the oracle: same token."""
    say("gumbel sampler extreme temperatures / logits V=151936")
    g = torch.Generator().manual_seed(14)
    R, V = 9, 151936
    lg = torch.randn((R, V), generator=g)
    for base in (0, 3, 6):
        lg[base + 1, 100] = float("inf")
        lg[base + 1, 200] = float("-inf")
        lg[base + 2, 50:60] = float("nan")
        lg[base + 2, 70000] = 3e38
        lg[base + 2, 70001] = -3e38
    temps = torch.tensor([1e-30, 1e-30, 1e-30, 1e30, 1e30, 1e30, 1.0, 1.0, 1.0], dtype=torch.float32)
    out = torch.empty(R, dtype=torch.int64, device=DEV)
    for seed, off in ((1, 0), (0xDEADBEEF12345678, 7)):
        ops.fused.sample_tokens(out, lg.to(DEV), None, temps.to(DEV), seed, off)
        torch.cuda.synchronize()
        want = orc.sample_tokens(lg.numpy(), temps=temps.numpy(), seed=seed, offset=off)
        got = out.cpu().numpy()
        assert np.array_equal(got, want), f"seed {seed}: got {got} want {want}"


def test_feed_tokens_and_embedding():
    say("feed_tokens / embedding")
    prev = torch.tensor([100, 101, 102, 103], dtype=torch.int64, device=DEV)
    tokens = torch.tensor([5, 6, 7, 8, 9], dtype=torch.int64, device=DEV)
    src = torch.tensor([-1, 3, -1, 0, 0], dtype=torch.int64, device=DEV)
    ops.fused.feed_tokens(tokens, src, prev)
    assert tokens.cpu().tolist() == [5, 103, 7, 100, 100]
    g = torch.Generator().manual_seed(13)
    table = torch.randn((1000, 1024), generator=g).to(torch.bfloat16).to(DEV)
    ids = torch.tensor([0, 999, 17, 17, -1, 1000], dtype=torch.int64, device=DEV)
    out = torch.empty((6, 1024), dtype=torch.bfloat16, device=DEV)
    ops.embedding(out, table, ids)
    torch.cuda.synchronize()
    assert torch.equal(out[:4], table[ids[:4]])
    assert torch.count_nonzero(out[4:]) == 0
