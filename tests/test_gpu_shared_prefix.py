"""Shared-prefix units of the planned decode launch (cvh_paged_attention_plan_shared + the _shared
launches) on the GPU, against the CPU oracle.

Sequences whose block tables start with the same physical blocks (prefix-cache hits,
engine/block_manager.cpp:80-116) are grouped by the plan; each group's shared keys are read once
per unit of up to 16 / GQA member tokens (one matrix-core pass over 16 query columns per kv head)
and each member's own tiles start after them; the merge combines the two. The result must equal
the oracle's attention over the whole context of every token (every row checked), be bitwise
reproducible, and agree with the plain planned launch within the attention tolerance (another
summation order). Edge cases: groups of 2, of 8 and of 19 members (three units), members whose
whole context lies in the shared blocks, a row that reports shared blocks but has no partner, a
padding token, 16- and 256-token blocks, per-tensor scales, a group cut across workgroup ranges
(explicit partition counts) and the split / merge phases."""
import math

import numpy as np
import pytest
import torch

from cppvllm_amd import _lib, ops, workloads
from tests._util import assert_close_bf16, bits, np_, say

pytestmark = pytest.mark.gpu
DEV = "cuda"


def run_oracle(orc, b):
    mode = orc.PER_TENSOR if b["k_scale"].numel() == 1 else orc.PER_TOKEN_HEAD
    return orc.paged_attention_fp8(np_(b["q"]), np_(b["k_cache"]), np_(b["v_cache"]), np_(b["k_scale"]),
                                   np_(b["v_scale"]), np_(b["block_tables"]), np_(b["token_seq"]),
                                   np_(b["token_kv_len"]), b["n_heads"], b["n_kv_heads"], b["head_dim"],
                                   b["block_size"], mode, b["scale"])


def run_planned(b, shared: bool, partitions: int = 0, phases: bool = False):
    T, H, HD = b["q"].shape
    KV, BS, W = b["n_kv_heads"], b["block_size"], b["block_tables"].shape[1]
    ws = ops.paged_attention_workspace(T, H, KV, HD, W, BS, partitions, DEV, shared=True)
    ops.paged_attention_plan(b["block_tables"], b["token_seq"], b["token_kv_len"], H, KV, HD, BS, ws, partitions,
                             shared_blocks=b["shared_blocks"] if shared else None)
    out = torch.full_like(b["q"], float("nan"))
    if phases:
        L = _lib.lib()
        mode = _lib.SCALE_PER_TENSOR if b["k_scale"].numel() == 1 else _lib.SCALE_PER_TOKEN_HEAD
        args = (out.data_ptr(), b["q"].data_ptr(), b["k_cache"].data_ptr(), b["v_cache"].data_ptr(),
                b["k_scale"].data_ptr(), b["v_scale"].data_ptr(), b["block_tables"].data_ptr(), W,
                b["token_seq"].data_ptr(), b["token_kv_len"].data_ptr(), T, H, KV, HD, BS, mode, b["scale"],
                partitions, ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
        assert L.cvh_paged_attention_fp8_planned_shared_split_phase(*args) == 0
        assert L.cvh_paged_attention_fp8_planned_shared_merge_phase(*args) == 0
    else:
        ops.paged_attention_fp8(out, b["q"], b["k_cache"], b["v_cache"], b["k_scale"], b["v_scale"],
                                b["block_tables"], b["token_seq"], b["token_kv_len"], b["scale"], workspace=ws,
                                partitions=partitions, planned=True, shared=shared)
    torch.cuda.synchronize()
    return bits(out)


def grouped_batch(seed, BS, groups, singles, per_tensor=False, pad=True, n_heads=16):
    """groups: list of (n_members, shared_blocks, [extra keys per member]); singles: context lengths
    of sequences that share nothing; one sequence reports shared blocks without a partner; a
    padding token (token_seq -1) at the end when pad."""
    g = torch.Generator().manual_seed(seed)
    rows, shared_cnt = [], []
    nb = 0
    for n, sb, extras in groups:
        prefix = list(range(nb, nb + sb))
        nb += sb
        for i in range(n):
            extra = extras[i % len(extras)]
            own = -(-max(extra - 0, 0) // BS) if extra > 0 else 0
            ctx = sb * BS + extra if extra >= 0 else sb * BS + extra   # extra < 0: context inside the prefix
            blocks = prefix + list(range(nb, nb + own))
            nb += own
            rows.append((blocks, ctx))
            shared_cnt.append(sb)
    for L in singles:
        k = -(-L // BS)
        rows.append((list(range(nb, nb + k)), L))
        nb += k
        shared_cnt.append(0)
    k = -(-700 // BS)                                   # claims 2 shared blocks, shares them with nobody
    rows.append((list(range(nb, nb + k)), 700))
    nb += k
    shared_cnt.append(2)
    perm = torch.randperm(nb + 2, generator=g).tolist()  # physical ids: a random permutation of the pool
    W = max(len(r[0]) for r in rows)
    table = torch.full((len(rows), W), -1, dtype=torch.int64)
    for i, (blocks, _) in enumerate(rows):
        table[i, :len(blocks)] = torch.tensor([perm[x] for x in blocks], dtype=torch.int64)
    x = torch.randn((nb + 2, BS, 8, 128), generator=g)
    y = torch.randn((nb + 2, BS, 8, 128), generator=g)
    kc, ks = workloads.quantize_blocks(x, per_tensor)
    vc, vs = workloads.quantize_blocks(y, per_tensor)
    # token order interleaves the groups with the other sequences
    order = torch.randperm(len(rows), generator=g).tolist()
    tseq = order + ([-1] if pad else [])
    tlen = [rows[i][1] for i in order] + ([50] if pad else [])
    T = len(tseq)
    q = torch.randn((T, n_heads, 128), generator=g).to(torch.bfloat16)
    return {"q": q, "k_cache": kc, "v_cache": vc, "k_scale": ks, "v_scale": vs, "block_tables": table,
            "token_seq": torch.tensor(tseq, dtype=torch.int64), "token_kv_len": torch.tensor(tlen, dtype=torch.int64),
            "shared_blocks": torch.tensor(shared_cnt, dtype=torch.int32), "block_size": BS, "n_heads": n_heads,
            "n_kv_heads": 8, "head_dim": 128, "scale": 1 / math.sqrt(128)}


def to_dev(b):
    return {k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in b.items()}


def test_config4b_units_all_rows(orc):
    """BASELINE config 4b (32 of 64 sequences share 8 blocks: 4 units of 8): all 64 rows vs the
    oracle, bitwise reproducible, within the tolerance of the plain planned launch."""
    say("config4b shared-prefix units: 64 rows vs oracle, reproducibility, vs plain plan")
    b = workloads.config4(device=DEV, shared_prefix=True)
    got = run_planned(b, True)
    assert np.array_equal(got, run_planned(b, True))
    cpu = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in b.items()}
    assert_close_bf16(got, run_oracle(orc, cpu), ulp_floor=True)
    plain = run_planned(b, False)
    assert_close_bf16(got, plain, ulp_floor=True)
    # the units ran: another summation order for the 32 sharing rows (the other rows' pieces move
    # too, since the member rows are shorter and the units join the tile space)
    shared_rows = np.nonzero(b["shared_blocks"].cpu().numpy() > 0)[0]
    assert not np.array_equal(got[shared_rows], plain[shared_rows])


@pytest.mark.parametrize("BS,per_tensor", [(256, False), (16, False), (16, True), (64, False)])
def test_units_grouped_batch(orc, BS, per_tensor):
    groups = [(2, 2, [40]), (8, 3, [1, 300, 17, 64]), (19, 1, [200, 5, 1000, 33, 0]),
              (4, 2, [-7, 10])]                          # -7: the whole context lies in the prefix
    say(f"shared-prefix units: groups of 2/8/19/2/2 members, BS={BS}, per_tensor={per_tensor}")
    b = grouped_batch(100 + BS + per_tensor, BS, groups, singles=[90, 2000, 1], per_tensor=per_tensor)
    want = run_oracle(orc, b)
    d = to_dev(b)
    got = run_planned(d, True)
    assert_close_bf16(got, want, ulp_floor=True)
    assert not got[-1].any(), "the padding token's row must be zero"
    assert np.array_equal(got, run_planned(d, True, phases=True))
    for parts in (3, 64, 700):                           # groups and units cut across ranges
        assert_close_bf16(run_planned(d, True, partitions=parts), want, ulp_floor=True)


@pytest.mark.parametrize("H", [8, 32, 64])
def test_units_other_gqa(orc, H):
    """GQA 1 / 4 / 8 at head_dim 128: units of 16 / 4 / 2 member tokens (16 matrix-core columns),
    groups of 2 to 19 members, whole and cut units, split / merge phases."""
    groups = [(2, 2, [40]), (3, 1, [7, 100, 0]), (8, 3, [1, 300, 17, 64]), (19, 1, [200, 5, 1000, 33, 0]),
              (4, 2, [-7, 10])]
    say(f"shared-prefix units at GQA {H // 8}: groups of 2/3/8/19/4 members")
    b = grouped_batch(300 + H, 64, groups, singles=[90, 2000, 1], n_heads=H)
    want = run_oracle(orc, b)
    d = to_dev(b)
    got = run_planned(d, True)
    assert_close_bf16(got, want, ulp_floor=True)
    assert not got[-1].any(), "the padding token's row must be zero"
    assert np.array_equal(got, run_planned(d, True))
    assert np.array_equal(got, run_planned(d, True, phases=True))
    plain = run_planned(d, False)
    ts = b["token_seq"].numpy()
    shared_rows = np.nonzero((ts >= 0) & (b["shared_blocks"].numpy()[ts.clip(0)] > 0))[0]
    assert not np.array_equal(got[shared_rows], plain[shared_rows]), "the units did not run"
    for parts in (3, 64, 700):
        assert_close_bf16(run_planned(d, True, partitions=parts), want, ulp_floor=True)


def test_units_respect_head_layout_limits(orc):
    """Shapes without the unit path (head_dim 64, kv heads in several row groups) accept the
    shared plan and run it as the plain one, matching the oracle."""
    say("shared plan on shapes without units (HD 64 GQA 2)")
    for HD, H in ((64, 16),):
        b = grouped_batch(7 + HD + H, 256, [(4, 2, [30, 500])], singles=[300])
        g = torch.Generator().manual_seed(HD + H)
        b["n_heads"], b["head_dim"], b["scale"] = H, HD, 1 / math.sqrt(HD)
        b["q"] = torch.randn((b["q"].shape[0], H, HD), generator=g).to(torch.bfloat16)
        x = torch.randn(b["k_cache"].shape[:3] + (HD,), generator=g)
        b["k_cache"], b["k_scale"] = workloads.quantize_blocks(x, False)
        b["v_cache"], b["v_scale"] = workloads.quantize_blocks(torch.randn_like(x), False)
        got = run_planned(to_dev(b), True)
        assert_close_bf16(got, run_oracle(orc, b), ulp_floor=True)


@pytest.mark.parametrize("seed,H", [(s, 16) for s in range(12)] + [(100 + s, h) for s in range(3) for h in (8, 32, 64)])
def test_units_random_groups(orc, seed, H):
    """Seeded random grouped batches: 1-5 groups of 2-20 members sharing 1-6 blocks with 0-2000 own
    keys (or a context inside the prefix), 0-20 other sequences, block size 16-1024, either scale
    mode, automatic or random partition counts, 8 / 16 / 32 / 64 query heads over 8 kv heads (units of
    16 / 8 / 4 / 2 tokens): every row against the oracle, reproducible."""
    r = np.random.default_rng(500 + seed)
    BS = int(r.choice([16, 32, 64, 256, 1024]))
    groups = []
    for _ in range(int(r.integers(1, 6))):
        sb = int(r.integers(1, 7))
        extras = [int(r.integers(-BS + 1, 0)) if r.random() < 0.15 else int(r.integers(0, 2001))
                  for _ in range(3)]
        groups.append((int(r.integers(2, 21)), sb, extras))
    singles = [int(r.integers(1, 3000)) for _ in range(int(r.integers(0, 21)))]
    per_tensor = bool(r.integers(2))
    parts = 0 if r.random() < 0.5 else int(r.integers(1, 500))
    say(f"random shared-prefix case seed={seed} H={H} BS={BS} groups={[(g[0], g[1]) for g in groups]} "
        f"singles={len(singles)} per_tensor={per_tensor} parts={parts}")
    b = grouped_batch(900 + seed, BS, groups, singles, per_tensor=per_tensor, n_heads=H)
    want = run_oracle(orc, b)
    d = to_dev(b)
    got = run_planned(d, True, partitions=parts)
    assert_close_bf16(got, want, ulp_floor=True)
    assert np.array_equal(got, run_planned(d, True, partitions=parts))
