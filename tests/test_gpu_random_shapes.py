"""Seeded random sweep of the attention entry points against the CPU oracle, through the C ABI.

Each case draws a head layout, block size (16-4096), scale mode, partition count and a ragged batch (1-40
sequences, contexts log-uniform in [1, 3000] keys, 1-3 trailing query tokens per sequence; or
100-300 sequences of one token with contexts up to 6000 keys), with a few empty or padding rows,
and checks: the plain decode launch against the oracle at the build's bar (max-abs 2e-2, mean-abs
2e-3), the planned launch bitwise equal to the plain one, and, where the multi-query kernel takes
the head layout, its plain and planned launches against the oracle.
The hand-picked cases in test_gpu_attention.py cover named boundaries; this sweep covers their
combinations."""
import math

import numpy as np
import pytest
import torch

from cppvllm_amd import ops
from tests._util import assert_close_bf16, say
from tests.test_gpu_attention import dev, run_gpu, run_oracle, run_planned, synth

pytestmark = pytest.mark.gpu

# (H, KV, HD) layouts the decode kernel takes (GQA 1/2/4/8, head_dim 64 and 128)
LAYOUTS = [(8, 8, 128), (16, 8, 128), (32, 8, 128), (64, 8, 128), (16, 8, 64), (8, 2, 64), (16, 4, 64),
           (64, 8, 64), (4, 4, 128), (2, 1, 128)]
BLOCK_SIZES = [16, 32, 64, 128, 256, 1024]


def draw(seed, wide=False):
    """wide: a decode-sized batch (100-300 sequences, one query token each, contexts up to 6000)."""
    r = np.random.default_rng(seed)
    H, KV, HD = LAYOUTS[r.integers(len(LAYOUTS))]
    sizes = BLOCK_SIZES if wide else BLOCK_SIZES + [2048, 4096]    # (wide batches: host memory)
    BS = int(sizes[r.integers(len(sizes))])
    n = int(r.integers(100, 301)) if wide else int(r.integers(1, 41))
    lens = [max(1, int(math.exp(r.uniform(0, math.log(6000 if wide else 3000))))) for _ in range(n)]
    qps = 1 if wide else int(r.integers(1, 4))
    per_tensor = bool(r.integers(2))
    parts = 0 if r.random() < 0.5 else int(r.integers(1, 600))
    b = synth(1000 + seed, lens, BS, H=H, KV=KV, HD=HD, per_tensor=per_tensor, queries_per_seq=qps)
    T = b["q"].shape[0]
    # a few rows with no context and, separately, padding rows (token_seq -1 with a kv_len): both
    # are zero rows in every entry point
    for t in r.choice(T, size=min(T, int(r.integers(0, 3))), replace=False):
        b["token_kv_len"][int(t)] = 0
    for t in r.choice(T, size=min(T, int(r.integers(0, 2))), replace=False):
        b["token_seq"][int(t)] = -1
    desc = f"seed={seed} H={H} KV={KV} HD={HD} BS={BS} seqs={n} T={T} qps={qps} per_tensor={per_tensor} parts={parts}"
    return b, parts, desc


@pytest.mark.parametrize("seed,wide", [(s, False) for s in range(48)] + [(s, True) for s in range(100, 112)])
def test_random_shapes_against_oracle(orc, seed, wide):
    b, parts, desc = draw(seed, wide)
    say(f"random attention case {desc}")
    want = run_oracle(orc, b)
    db = dev(b)
    got = run_gpu(db, parts)
    assert_close_bf16(got, want, ulp_floor=True)
    assert np.array_equal(run_planned(db, parts), got), "planned launch differs from the plain launch"
    H, KV, HD = b["n_heads"], b["n_kv_heads"], b["head_dim"]
    if ops.prefill_supported(H, KV, HD):
        for mode in (True, "planned"):
            say(f"random attention case {desc} multi-query mode={mode}")
            assert_close_bf16(run_gpu(db, prefill=mode), want, ulp_floor=True)
