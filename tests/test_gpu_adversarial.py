"""GPU parity on adversarial caches: 1% of K/V values at 20x (config 4's outliers) with every
attention path (VALU decode, MFMA decode at GQA 8, virtual kv heads at head_dim 64, the
one-kv-head packed launch, the prefill kernel plain and planned), per-tensor and per-(token, head)
scales, 16- to 256-token blocks, and peaked softmax (q scaled by 4 or 8). All rows against the
oracle at the one-ulp floor (outputs reach |x| ~ 90); decode planned == plain bitwise."""
import math

import numpy as np
import pytest
import torch

from cppvllm_amd import workloads
from tests._util import assert_close_bf16, say
from tests.test_gpu_attention import run_gpu, run_oracle, run_planned, dev

pytestmark = pytest.mark.gpu


def synth_outliers(seed, lens, BS, H, KV, HD, per_tensor, q_mult, queries_per_seq=1):
    """Random block tables and N(0,1) K/V with 1% of values at 20x, quantised to e4m3; q scaled
    by q_mult; queries_per_seq > 1 gives chunked-prefill rows (the last positions of each context)."""
    g = torch.Generator().manual_seed(seed)
    nblk = [math.ceil(L / BS) for L in lens]
    nb = sum(nblk) + 2
    perm = torch.randperm(nb, generator=g)
    table = torch.full((len(lens), max(nblk)), -1, dtype=torch.int64)
    p = 0
    for i, n in enumerate(nblk):
        table[i, :n] = perm[p:p + n]
        p += n
    def kv():
        x = torch.randn((nb, BS, KV, HD), generator=g)
        return torch.where(torch.rand(x.shape, generator=g) < 0.01, x * 20.0, x)
    kc, ks = workloads.quantize_blocks(kv(), per_tensor)
    vc, vs = workloads.quantize_blocks(kv(), per_tensor)
    tseq, tlen = [], []
    for i, L in enumerate(lens):
        for j in range(min(queries_per_seq, L)):
            tseq.append(i)
            tlen.append(L - j)
    q = (torch.randn((len(tseq), H, HD), generator=g) * q_mult).to(torch.bfloat16)
    return {"q": q, "k_cache": kc, "v_cache": vc, "k_scale": ks, "v_scale": vs, "block_tables": table,
            "token_seq": torch.tensor(tseq, dtype=torch.int64), "token_kv_len": torch.tensor(tlen, dtype=torch.int64),
            "block_size": BS, "n_heads": H, "n_kv_heads": KV, "head_dim": HD, "scale": 1 / math.sqrt(HD)}


LENS = [3000, 1200, 4500, 700, 33, 2048, 1, 257]


@pytest.mark.parametrize("BS,H,KV,HD,per_tensor,q_mult", [
    (16, 16, 8, 128, False, 1), (16, 16, 8, 128, True, 1), (256, 64, 8, 128, True, 1), (32, 64, 8, 64, False, 1),
    (256, 16, 8, 128, False, 8), (256, 64, 8, 128, False, 8), (64, 32, 8, 128, False, 4), (256, 2, 1, 128, False, 1)])
def test_decode_adversarial(orc, BS, H, KV, HD, per_tensor, q_mult):
    say(f"decode adversarial BS={BS} H={H} KV={KV} HD={HD} pt={per_tensor} q*{q_mult}")
    b = synth_outliers(BS + H + HD + q_mult, LENS, BS, H, KV, HD, per_tensor, q_mult)
    want = run_oracle(orc, b)
    db = dev(b)
    got = run_gpu(db)
    assert_close_bf16(got, want, ulp_floor=True)
    assert np.array_equal(run_planned(db), got)


@pytest.mark.parametrize("mode", [True, "planned"])
@pytest.mark.parametrize("BS,per_tensor,q_mult", [(16, False, 1), (256, True, 1), (256, False, 8), (32, False, 4)])
def test_prefill_adversarial(orc, BS, per_tensor, q_mult, mode):
    say(f"prefill adversarial BS={BS} pt={per_tensor} q*{q_mult} {mode}")
    b = synth_outliers(7 + BS + q_mult, [3000, 1200, 700, 130], BS, 16, 8, 128, per_tensor, q_mult, queries_per_seq=100)
    want = run_oracle(orc, b)
    got = run_gpu(dev(b), prefill=mode)
    assert_close_bf16(got, want, ulp_floor=True)
