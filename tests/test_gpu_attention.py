"""GPU parity of the FP8 paged decode attention against the CPU oracle, through the C ABI.

Bar: max-abs 2e-2 and mean-abs 2e-3 on the bf16 outputs (the build's stated tolerance).
Covers BASELINE configs 1 (both scale modes), 3 (full headline size), 4 and 4b (long contexts,
split-K, shared prefix blocks, outliers), the reference's 16-token blocks, GQA ratios 1/2/4/8,
head_dim 64, ragged and boundary lengths, chunked-prefill continuation rows, empty contexts,
split-count invariance and physical-block permutation invariance, block sizes 16 to 4096 and the
query-token limits of the GQA 4/8 virtual kv heads."""
import math

import numpy as np
import pytest
import torch

from cppvllm_amd import _lib, ops, workloads
from tests._util import assert_close_bf16, bits, np_, say

pytestmark = pytest.mark.gpu
DEV = "cuda"


def run_gpu(b, partitions=0, prefill=False):
    """prefill: False (decode kernel), True (multi-query kernel) or "planned" (its planned launch)."""
    out = torch.empty_like(b["q"])
    if prefill:
        pws = None
        if prefill == "planned":
            pws = ops.prefill_workspace(b["q"].shape[0], b["q"].device)
            ops.paged_attention_prefill_plan(b["token_seq"], b["token_kv_len"], b["block_tables"].shape[1],
                                             b["block_size"], pws)
        ops.paged_attention_fp8_prefill(out, b["q"], b["k_cache"], b["v_cache"], b["k_scale"], b["v_scale"],
                                        b["block_tables"], b["token_seq"], b["token_kv_len"], b["scale"],
                                        workspace=pws)
    else:
        ops.paged_attention_fp8(out, b["q"], b["k_cache"], b["v_cache"], b["k_scale"], b["v_scale"],
                                b["block_tables"], b["token_seq"], b["token_kv_len"], b["scale"],
                                partitions=partitions)
    torch.cuda.synchronize()
    return bits(out)


def run_oracle(orc, b, rows=None):
    H, KV, HD, BS = b["n_heads"], b["n_kv_heads"], b["head_dim"], b["block_size"]
    mode = orc.PER_TENSOR if b["k_scale"].numel() == 1 else orc.PER_TOKEN_HEAD
    tseq, tlen, q = np_(b["token_seq"]), np_(b["token_kv_len"]), np_(b["q"])
    if rows is not None:
        tseq, tlen, q = tseq[rows].copy(), tlen[rows].copy(), q[rows].copy()
    return orc.paged_attention_fp8(q, np_(b["k_cache"]), np_(b["v_cache"]), np_(b["k_scale"]), np_(b["v_scale"]),
                                   np_(b["block_tables"]), tseq, tlen, H, KV, HD, BS, mode, b["scale"])


def synth(seed, lens, BS, H=16, KV=8, HD=128, per_tensor=False, queries_per_seq=1):
    """Random quantised cache + q; optional several query tokens per sequence (chunked prefill:
    the last `queries_per_seq` positions of each context, causal kv_len = pos + 1)."""
    g = torch.Generator().manual_seed(seed)
    nblk = [math.ceil(L / BS) for L in lens]
    nb = sum(nblk) + 3
    perm = torch.randperm(nb, generator=g)
    W = max(nblk)
    table = torch.full((len(lens), W), -1, dtype=torch.int64)
    p = 0
    for i, n in enumerate(nblk):
        table[i, :n] = perm[p:p + n]
        p += n
    x = torch.randn((nb, BS, KV, HD), generator=g)
    y = torch.randn((nb, BS, KV, HD), generator=g)
    kc, ks = workloads.quantize_blocks(x, per_tensor)
    vc, vs = workloads.quantize_blocks(y, per_tensor)
    tseq, tlen = [], []
    for i, L in enumerate(lens):
        for j in range(min(queries_per_seq, L)):
            tseq.append(i)
            tlen.append(L - j)
    T = len(tseq)
    q = torch.randn((T, H, HD), generator=g).to(torch.bfloat16)
    b = {"q": q, "k_cache": kc, "v_cache": vc, "k_scale": ks, "v_scale": vs, "block_tables": table,
         "token_seq": torch.tensor(tseq, dtype=torch.int64), "token_kv_len": torch.tensor(tlen, dtype=torch.int64),
         "block_size": BS, "n_heads": H, "n_kv_heads": KV, "head_dim": HD, "scale": 1 / math.sqrt(HD)}
    return b


def dev(b):
    return {k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in b.items()}


@pytest.mark.parametrize("per_tensor", [True, False])
def test_config1(orc, per_tensor):
    say(f"config1 per_tensor={per_tensor}")
    b = workloads.config1(device="cpu", per_tensor=per_tensor)
    want = run_oracle(orc, b)
    got = run_gpu(dev(b))
    assert_close_bf16(got, want)


@pytest.mark.parametrize("BS,H,KV,HD,per_tensor", [
    (16, 16, 8, 128, False), (16, 16, 8, 128, True), (256, 16, 8, 128, False), (32, 8, 8, 128, False),
    (64, 32, 8, 128, False), (16, 64, 8, 128, False), (16, 8, 2, 64, False), (128, 16, 4, 64, True),
    (4096, 16, 8, 128, False), (1024, 32, 8, 128, False), (512, 64, 8, 64, True), (2048, 8, 8, 128, False),
])
def test_shapes_and_boundaries(orc, BS, H, KV, HD, per_tensor):
    lens = [1, 2, 15, 16, 17, 31, 32, 33, 63, 64, 65, 255, 256, 257, 511, 777, 1030]
    say(f"shapes BS={BS} H={H} KV={KV} HD={HD} per_tensor={per_tensor}")
    b = synth(BS * 7 + H + KV + HD, lens, BS, H, KV, HD, per_tensor)
    want = run_oracle(orc, b)
    got = run_gpu(dev(b))
    assert_close_bf16(got, want)


@pytest.mark.parametrize("split", [1, 2, 7, 64, 511, 4096])
def test_partition_invariance(orc, split):
    say(f"partition invariance partitions={split}")
    b = synth(11, [70, 600, 1500, 2100, 3000], 16)
    db = dev(b)
    base = run_gpu(db, 0)
    got = run_gpu(db, split)
    assert_close_bf16(got, base, max_abs=8e-3, mean_abs=5e-4)
    assert_close_bf16(got, run_oracle(orc, b))


def test_chunked_prefill_rows(orc):
    say("chunked prefill continuation rows")
    b = synth(21, [40, 300, 1000], 16, queries_per_seq=37)
    assert_close_bf16(run_gpu(dev(b)), run_oracle(orc, b))


def test_max_rows_per_launch(orc):
    # 8192 query tokens x 8 kv heads = 8192 rows, the per-launch limit (LDS above 64 KiB);
    # the oracle checks a seeded sample of 192 rows
    say("max rows per launch: 8 seqs x 1024 chunked-prefill tokens")
    b = synth(41, [1024, 1100, 1500, 2000, 1024, 1300, 1700, 1900], 256, queries_per_seq=1024)
    assert b["q"].shape[0] == 8192
    got = run_gpu(dev(b))
    rows = sorted(np.random.default_rng(41).choice(8192, 192, replace=False).tolist())
    assert_close_bf16(got[rows], run_oracle(orc, b, rows=rows))


def test_partition_bounds_past_32_bits(orc):
    """Tiles x partitions above 2^32: the merge's range bounds take the 64-bit division (32-bit
    below); the result must match the automatic partition count's and the oracle's sampled rows."""
    b = synth(41, [1024, 1100, 1500, 2000, 1024, 1300, 1700, 1900], 256, queries_per_seq=1024)
    U = int(sum((int(k) + 31) // 32 for k in np_(b["token_kv_len"])))
    G = (1 << 32) // U + 64
    assert (U + 1) * G > (1 << 32)
    say(f"partition bounds past 32 bits: U={U} G={G}")
    db = dev(b)
    got = run_gpu(db, G)
    assert_close_bf16(got, run_gpu(db, 0), max_abs=8e-3, mean_abs=5e-4)
    rows = sorted(np.random.default_rng(47).choice(8192, 96, replace=False).tolist())
    assert_close_bf16(got[rows], run_oracle(orc, b, rows=rows))


@pytest.mark.parametrize("H,HD,limit", [(32, 64, 4096), (64, 64, 2048), (64, 128, 8192)])
def test_gqa_row_limits(orc, H, HD, limit):
    """At head_dim 64, GQA 4 / 8 run as 2 / 4 virtual kv heads per kv head, so at 8 kv heads a
    launch takes at most 4096 / 2048 query tokens; at head_dim 128 they run on MFMA with one wave
    per kv head and take the full 8192. The limit itself is computed (sampled rows vs the oracle),
    one more token per sequence is rejected with CVH_ERR_UNSUPPORTED before anything runs."""
    say(f"GQA row limit H={H} HD={HD} T={limit}")
    per = limit // 4
    b = synth(43 + H + HD, [per + 50, per + 300, per + 7, per + 999], 256, H=H, HD=HD, queries_per_seq=per)
    assert b["q"].shape[0] == limit
    got = run_gpu(dev(b))
    rows = sorted(np.random.default_rng(H + HD).choice(limit, 96, replace=False).tolist())
    assert_close_bf16(got[rows], run_oracle(orc, b, rows=rows))
    b1 = dev(synth(44 + H + HD, [per + 50, per + 300, per + 7, per + 999], 256, H=H, HD=HD,
                   queries_per_seq=per + 1))
    assert b1["q"].shape[0] == limit + 4
    with pytest.raises(_lib.CvhError) as err:
        run_gpu(b1)
    assert err.value.code == _lib.CVH_ERR_UNSUPPORTED


@pytest.mark.parametrize("H", [32, 64])
def test_gqa_mfma_config3_and_planned(orc, H):
    """GQA 4 / 8 on the MFMA path at the headline shape (config-3 K/V, 256 sequences, 256-token
    blocks): oracle parity on sampled rows, planned == unplanned bitwise, and every head equals
    the same head computed by the GQA-2 (VALU) kernel: query heads 2i, 2i+1 of each kv head's
    group go through a GQA-2 launch of their own, so two independent kernels agree on all rows."""
    say(f"GQA MFMA config 3 H={H}")
    b = workloads.config3(device="cpu")
    g = torch.Generator().manual_seed(H)
    rep = H // 8
    b["n_heads"] = H
    b["q"] = torch.randn((b["q"].shape[0], H, 128), generator=g).to(torch.bfloat16)
    db = dev(b)
    got = run_gpu(db)
    rows = list(range(0, 256, 9))
    assert_close_bf16(got[rows], run_oracle(orc, b, rows=rows))
    assert np.array_equal(run_planned(db), got)
    q8 = db["q"].view(256, 8, rep, 128)
    for i in range(rep // 2):
        d2 = dict(db)
        d2["n_heads"] = 16
        d2["q"] = q8[:, :, 2 * i:2 * i + 2].reshape(256, 16, 128).contiguous()
        two = run_gpu(d2).reshape(256, 8, 2, 128)
        mine = got.reshape(256, 8, rep, 128)[:, :, 2 * i:2 * i + 2]
        assert_close_bf16(mine, two, max_abs=1.6e-2, mean_abs=1e-3)


@pytest.mark.parametrize("H", [32, 64])
def test_gqa_mfma_config4_outliers(orc, H):
    """GQA 4 / 8 on the MFMA path over config 4 (contexts to 32k keys, 20x outliers): all 64 rows
    against the oracle. The outputs reach |x| ~ 60, so the bar is the one-ulp floor of
    test_config4_long_context; the PV weights must carry more than one bf16 rounding for it."""
    say(f"GQA MFMA config 4 H={H}")
    b = workloads.config4(device="cpu")
    g = torch.Generator().manual_seed(H)
    b["n_heads"] = H
    b["q"] = torch.randn((b["q"].shape[0], H, 128), generator=g).to(torch.bfloat16)
    got = run_gpu(dev(b))
    assert_close_bf16(got, run_oracle(orc, b), ulp_floor=True)


def test_empty_context_rows_are_zero(orc):
    say("kv_len 0 rows")
    b = synth(5, [100, 50], 16)
    b["token_kv_len"][1] = 0
    got = run_gpu(dev(b))
    assert (got[1] == 0).all()
    assert_close_bf16(got[:1], run_oracle(orc, b, rows=[0]))


@pytest.mark.parametrize("mode", ["plain", "planned", "partitions_64"])
def test_padding_rows_are_zero(orc, mode):
    """token_seq < 0 marks a padding token: its output row is zero whatever its kv_len says (the
    same rule as the prefill kernel and the oracle), and the other rows are unaffected."""
    say(f"padding rows (token_seq -1, kv_len > 0): {mode}")
    b = synth(6, [300, 50, 1000, 700, 17], 16)
    b["token_seq"][1] = -1
    b["token_seq"][3] = -1
    b["token_kv_len"][3] = 4000          # beyond any table row: must not matter either
    db = dev(b)
    if mode == "planned":
        got = run_planned(db)
    else:
        got = run_gpu(db, 64 if mode == "partitions_64" else 0)
    assert not got[1].any() and not got[3].any()
    assert_close_bf16(got, run_oracle(orc, b))
    keep = [0, 2, 4]
    b2 = {k: v for k, v in b.items()}
    b2["q"], b2["token_seq"], b2["token_kv_len"] = b["q"][keep], b["token_seq"][keep], b["token_kv_len"][keep]
    assert_close_bf16(got[keep], run_gpu(dev(b2)), max_abs=8e-3, mean_abs=5e-4)


def test_block_permutation_invariance_bitwise():
    say("physical block permutation invariance")
    b = synth(31, [500, 900, 17], 16)
    base = run_gpu(dev(b))
    nb = b["k_cache"].shape[0]
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(1))
    inv = torch.argsort(perm)
    b2 = dict(b)
    for k in ("k_cache", "v_cache", "k_scale", "v_scale"):
        b2[k] = b[k][inv].contiguous()
    t = b["block_tables"]
    b2["block_tables"] = torch.where(t >= 0, perm[t.clamp_min(0)], t)
    assert np.array_equal(run_gpu(dev(b2)), base)


def test_config3_full(orc):
    say("config3 full: 256 seqs, BS=256, per-token scales")
    b = workloads.config3(device="cpu")
    want = run_oracle(orc, b)
    got = run_gpu(dev(b))
    say("config3 errors (max, mean):", assert_close_bf16(got, want))


@pytest.mark.parametrize("shared", [False, True])
def test_config4_long_context(orc, shared):
    say(f"config4 64 seqs log-U(4k,32k) shared_prefix={shared}")
    b = workloads.config4(device=DEV, shared_prefix=shared)
    got = run_gpu(b)
    assert np.isfinite((got.astype(np.uint32) << 16).view(np.float32)).all()
    bc = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in b.items()}
    # all 64 rows; outputs dominated by 20x outliers reach |x| > 4, where one bf16 ulp exceeds
    # 2e-2 and a value near a rounding midpoint legitimately rounds either way (row 43 of the
    # unshared case: exact -17.436, GPU -17.375, oracle -17.5)
    assert_close_bf16(got, run_oracle(orc, bc), ulp_floor=True)
    if shared:
        t = bc["block_tables"]
        assert (t[0, :8] == t[2, :8]).all() and (t[0, :8] == t[62, :8]).all()


def test_workspace_contract():
    say("workspace contract")
    from cppvllm_amd import _lib
    b = dev(synth(3, [3000, 20], 16))
    T, H = b["q"].shape[:2]
    W = b["block_tables"].shape[1]
    need = _lib.lib().cvh_paged_attention_workspace_bytes(T, H, 8, 128, W, 16, 64)
    assert need > 0
    small = torch.empty(need - 4, dtype=torch.uint8, device=DEV)
    with pytest.raises(_lib.CvhError) as e:
        ops.paged_attention_fp8(torch.empty_like(b["q"]), b["q"], b["k_cache"], b["v_cache"], b["k_scale"],
                                b["v_scale"], b["block_tables"], b["token_seq"], b["token_kv_len"], b["scale"],
                                workspace=small, partitions=64)
    assert e.value.code == _lib.CVH_ERR_WORKSPACE


def test_workspace_reused():
    say("workspace reuse: two calls with one workspace")
    from cppvllm_amd import _lib
    b = dev(synth(41, [3000, 700, 64, 1500], 16))
    T, H = b["q"].shape[:2]
    W = b["block_tables"].shape[1]
    ws = ops.paged_attention_workspace(T, H, 8, 128, W, 16, 64, DEV)
    outs = []
    for _ in range(2):
        out = torch.empty_like(b["q"])
        ops.paged_attention_fp8(out, b["q"], b["k_cache"], b["v_cache"], b["k_scale"], b["v_scale"],
                                b["block_tables"], b["token_seq"], b["token_kv_len"], b["scale"], workspace=ws,
                                partitions=64)
        torch.cuda.synchronize()
        outs.append(bits(out))
    assert np.array_equal(outs[0], outs[1])
    _ = _lib  # noqa


def test_graph_replay_matches_eager():
    say("hip graph capture + 3 replays")
    b = dev(synth(43, [900, 2500, 40, 333], 16))
    T, H = b["q"].shape[:2]
    W = b["block_tables"].shape[1]
    ws = ops.paged_attention_workspace(T, H, 8, 128, W, 16, 0, DEV)
    eager = run_gpu(b)
    out = torch.empty_like(b["q"])
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):   # warm-up on the capture stream
        ops.paged_attention_fp8(out, b["q"], b["k_cache"], b["v_cache"], b["k_scale"], b["v_scale"],
                                b["block_tables"], b["token_seq"], b["token_kv_len"], b["scale"], workspace=ws)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.paged_attention_fp8(out, b["q"], b["k_cache"], b["v_cache"], b["k_scale"], b["v_scale"],
                                b["block_tables"], b["token_seq"], b["token_kv_len"], b["scale"], workspace=ws)
    for i in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(out), eager), f"replay {i} differs from eager"
        _ = run_gpu(b)   # eager work between replays


def test_prefill_plan_and_kernel_graph_replay():
    """The prefill plan and the planned multi-query launch captured in one HIP graph (as the engine
    runs prompt steps): every replay, with new q, token lengths and eager work in between, equals
    the eager launch on the same inputs."""
    say("prefill plan + planned kernel: graph capture + 3 replays")
    b = dev(synth_prefill(44, [(300, 300), (1000, 70), (40, 40), (700, 129)], 16))
    T = b["q"].shape[0]
    pws = ops.prefill_workspace(T, DEV)
    out = torch.empty_like(b["q"])

    def body():
        ops.paged_attention_prefill_plan(b["token_seq"], b["token_kv_len"], b["block_tables"].shape[1],
                                         b["block_size"], pws)
        ops.paged_attention_fp8_prefill(out, b["q"], b["k_cache"], b["v_cache"], b["k_scale"], b["v_scale"],
                                        b["block_tables"], b["token_seq"], b["token_kv_len"], b["scale"],
                                        workspace=pws)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):   # warm-up on the capture stream
        body()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        body()
    gen = torch.Generator().manual_seed(45)
    kvl0 = b["token_kv_len"].clone()
    for i in range(3):
        b["q"].copy_(torch.randn(b["q"].shape, generator=gen).to(torch.bfloat16))
        b["token_kv_len"].copy_((kvl0 - i * 7).clamp_min(0))     # new lengths: the plan must follow them
        eager = run_gpu(b, prefill="planned")
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(out), eager), f"replay {i} differs from eager"


def test_split_and_merge_phases_equal_combined_call():
    say("split phase + merge phase == combined call")
    from cppvllm_amd import _lib
    b = dev(synth(47, [3000, 100, 1400], 16))
    T, H = b["q"].shape[:2]
    W = b["block_tables"].shape[1]
    ws = ops.paged_attention_workspace(T, H, 8, 128, W, 16, 64, DEV)
    base = run_gpu(b, 64)
    out = torch.empty_like(b["q"])
    args = (out.data_ptr(), b["q"].data_ptr(), b["k_cache"].data_ptr(), b["v_cache"].data_ptr(),
            b["k_scale"].data_ptr(), b["v_scale"].data_ptr(), b["block_tables"].data_ptr(), W,
            b["token_seq"].data_ptr(), b["token_kv_len"].data_ptr(), T, H, 8, 128, 16, 0, b["scale"], 64,
            ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
    lib = _lib.lib()
    assert lib.cvh_paged_attention_fp8_split_phase(*args) == 0
    assert lib.cvh_paged_attention_fp8_merge_phase(*args) == 0
    torch.cuda.synchronize()
    assert np.array_equal(bits(out), base)


def run_planned(b, partitions=0, ws=None):
    T, H, HD = b["q"].shape
    KV, BS, W = b["n_kv_heads"], b["block_size"], b["block_tables"].shape[1]
    if ws is None:
        ws = ops.paged_attention_workspace(T, H, KV, HD, W, BS, partitions, DEV)
        ops.paged_attention_plan(b["block_tables"], b["token_seq"], b["token_kv_len"], H, KV, HD, BS, ws, partitions)
    out = torch.empty_like(b["q"])
    ops.paged_attention_fp8(out, b["q"], b["k_cache"], b["v_cache"], b["k_scale"], b["v_scale"], b["block_tables"],
                            b["token_seq"], b["token_kv_len"], b["scale"], workspace=ws, partitions=partitions,
                            planned=True)
    torch.cuda.synchronize()
    return bits(out)


def _planned_case(name):
    if name == "config1_per_tensor":
        return workloads.config1(device="cpu", per_tensor=True), 0
    if name == "bs16_two_block_tiles":
        return synth(61, [40, 300, 1000, 17, 33], 16), 0
    if name == "chunked_prefill":
        return synth(62, [40, 300, 1000], 16, queries_per_seq=37), 0
    if name == "empty_rows":
        b = synth(63, [100, 50, 700, 1], 256)
        b["token_kv_len"][1] = 0
        return b, 0
    if name == "partitions_7":
        return synth(64, [3000, 100, 1400], 16), 7
    if name == "partitions_511":
        return synth(65, [3000, 100, 1400, 64], 64), 511
    if name == "gqa4_hd64":
        return synth(66, [500, 900], 32, H=16, KV=4, HD=64), 0
    raise KeyError(name)


@pytest.mark.parametrize("name", ["config1_per_tensor", "bs16_two_block_tiles", "chunked_prefill", "empty_rows",
                                  "partitions_7", "partitions_511", "gqa4_hd64"])
def test_planned_equals_unplanned_bitwise(name):
    say(f"planned == unplanned: {name}")
    b, parts = _planned_case(name)
    db = dev(b)
    assert np.array_equal(run_planned(db, parts), run_gpu(db, parts))


@pytest.mark.parametrize("parts", [0, 1028, 514, 1030, 1024])
def test_one_kv_head_packed_workgroups(orc, parts):
    """One kv head per row group: the launch runs 4 (or 2) tile ranges per workgroup when that
    leaves a workgroup per CU (automatic 1024 partitions -> 4; 1028 -> 4; 514, 1030 -> 2). Planned
    and unplanned launches agree bitwise, empty rows stay zero and sampled rows match the oracle."""
    say(f"one kv head, packed ranges, partitions {parts}")
    rng = np.random.default_rng(67)
    lens = [int(x) for x in rng.integers(1, 1400, size=200)]
    b = synth(67, lens, 16, H=2, KV=1)
    b["token_kv_len"][::17] = 0
    db = dev(b)
    got = run_gpu(db, parts)
    assert np.array_equal(run_planned(db, parts), got)
    assert not got[::17].any()
    rows = np.arange(1, 200, 13)
    assert_close_bf16(got[rows], run_oracle(orc, b, rows))


def test_plan_shared_by_layers_config3(orc):
    # one plan, two layers with different caches (the decode-step pattern); each equals the
    # unplanned call bitwise, and layer 0 matches the oracle
    say("config3: one plan, two layers")
    b = workloads.config3(device=DEV)
    T, H, HD = b["q"].shape
    KV, BS, W = b["n_kv_heads"], b["block_size"], b["block_tables"].shape[1]
    ws = ops.paged_attention_workspace(T, H, KV, HD, W, BS, 0, DEV)
    ops.paged_attention_plan(b["block_tables"], b["token_seq"], b["token_kv_len"], H, KV, HD, BS, ws)
    b2 = dict(b)
    g = torch.Generator(device=DEV).manual_seed(5)
    b2["k_cache"] = torch.randint(0, 126, b["k_cache"].shape, dtype=torch.uint8, device=DEV, generator=g)
    b2["v_cache"] = torch.randint(0, 126, b["v_cache"].shape, dtype=torch.uint8, device=DEV, generator=g)
    got1 = run_planned(b, ws=ws)
    got2 = run_planned(b2, ws=ws)
    assert np.array_equal(got1, run_gpu(b))
    assert np.array_equal(got2, run_gpu(b2))
    assert not np.array_equal(got1, got2)
    rows = list(range(0, T, 16))
    cpu = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in b.items()}
    assert_close_bf16(got1[rows], run_oracle(orc, cpu, rows=rows))


def test_planned_repeated_graph_launches():
    """One plan, 28 planned launches alternating two different caches in a HIP graph, replayed
    with eager work in between: every output equals the unplanned call bitwise, so no launch
    reads another launch's partials or plan state."""
    say("planned: 28 launches x 4 graph replays, alternating caches")
    b = workloads.config3(device=DEV, seqs=128)
    T, H, HD = b["q"].shape
    KV, BS, W = b["n_kv_heads"], b["block_size"], b["block_tables"].shape[1]
    b2 = dict(b)
    g = torch.Generator(device=DEV).manual_seed(7)
    b2["k_cache"] = torch.randint(0, 126, b["k_cache"].shape, dtype=torch.uint8, device=DEV, generator=g)
    b2["v_cache"] = torch.randint(0, 126, b["v_cache"].shape, dtype=torch.uint8, device=DEV, generator=g)
    want = [run_gpu(b), run_gpu(b2)]
    assert not np.array_equal(want[0], want[1])
    ws = ops.paged_attention_workspace(T, H, KV, HD, W, BS, 0, DEV)
    ops.paged_attention_plan(b["block_tables"], b["token_seq"], b["token_kv_len"], H, KV, HD, BS, ws)
    outs = [torch.empty_like(b["q"]) for _ in range(28)]

    def layers():
        for i, o in enumerate(outs):
            c = b if i % 2 == 0 else b2
            ops.paged_attention_fp8(o, c["q"], c["k_cache"], c["v_cache"], c["k_scale"], c["v_scale"],
                                    c["block_tables"], c["token_seq"], c["token_kv_len"], c["scale"], workspace=ws,
                                    planned=True)
    layers()
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        assert np.array_equal(bits(o), want[i % 2]), f"eager launch {i}"
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            layers()
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(4):
        for o in outs:
            o.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for i, o in enumerate(outs):
            assert np.array_equal(bits(o), want[i % 2]), f"replay {rep} launch {i}"
        assert np.array_equal(run_gpu(b2), want[1])          # eager work between replays


# ---- the MFMA multi-query (chunked-prefill) kernel -------------------------------------------------
def synth_prefill(seed, chunks, BS, H=16, KV=8, per_tensor=False, order="asc"):
    """chunks: (context length L, query tokens n) per sequence -> the n last positions of each
    context as consecutive query tokens (causal kv_len = pos + 1), in ascending (prefill order)
    or descending position order."""
    lens = [L for L, _ in chunks]
    b = synth(seed, lens, BS, H=H, KV=KV, per_tensor=per_tensor)
    tseq, tlen = [], []
    for i, (L, n) in enumerate(chunks):
        ks = range(L - n + 1, L + 1) if order == "asc" else range(L, L - n, -1)
        for k in ks:
            tseq.append(i)
            tlen.append(k)
    g = torch.Generator().manual_seed(seed + 1)
    b["q"] = torch.randn((len(tseq), H, 128), generator=g).to(torch.bfloat16)
    b["token_seq"] = torch.tensor(tseq, dtype=torch.int64)
    b["token_kv_len"] = torch.tensor(tlen, dtype=torch.int64)
    return b


PREFILL_MODES = [True, "planned"]


@pytest.mark.parametrize("mode", PREFILL_MODES)
@pytest.mark.parametrize("BS", [16, 32, 256])
@pytest.mark.parametrize("per_tensor", [False, True])
def test_prefill_kernel_matches_oracle(orc, BS, per_tensor, mode):
    say(f"prefill MFMA kernel BS={BS} per_tensor={per_tensor} mode={mode}")
    chunks = [(5, 5), (40, 40), (300, 300), (1000, 37), (17, 1), (700, 129), (2, 2)]
    b = synth_prefill(51 + BS, chunks, BS, per_tensor=per_tensor)
    assert_close_bf16(run_gpu(dev(b), prefill=mode), run_oracle(orc, b))


@pytest.mark.parametrize("mode", PREFILL_MODES)
@pytest.mark.parametrize("H,KV", [(8, 8), (16, 8), (4, 2), (2, 1), (32, 16)])
def test_prefill_kernel_head_layouts(orc, H, KV, mode):
    say(f"prefill MFMA kernel H={H} KV={KV} mode={mode}")
    b = synth_prefill(61 + H + KV, [(100, 100), (333, 60), (64, 16)], 16, H=H, KV=KV)
    assert_close_bf16(run_gpu(dev(b), prefill=mode), run_oracle(orc, b))


@pytest.mark.parametrize("mode", PREFILL_MODES)
def test_prefill_kernel_outlier_rows(orc, mode):
    """Chunked-prefill rows (the last 96 positions of 4 sequences, contexts to 5000) over a cache
    with config 4's 1% of 20x outliers: all rows against the oracle at the one-ulp floor (outputs
    reach |x| ~ 30, where the PV weights need more than bf16's 8 significant bits)."""
    say(f"prefill rows over outlier K/V, mode {mode}")
    lens = [3000, 1500, 800, 5000]
    b = workloads.decode_batch(lens, 256, 77, "cpu", outlier_frac=0.01)
    tseq, tlen = [], []
    for i, L in enumerate(lens):
        for j in range(96):
            tseq.append(i)
            tlen.append(L - 95 + j)
    b["token_seq"] = torch.tensor(tseq, dtype=torch.int64)
    b["token_kv_len"] = torch.tensor(tlen, dtype=torch.int64)
    b["q"] = torch.randn((len(tseq), 16, 128), generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    got = run_gpu(dev(b), prefill=mode)
    assert_close_bf16(got, run_oracle(orc, b), ulp_floor=True)


def test_prefill_plan_orders_groups_longest_first():
    """The plan is a permutation of the 64-token groups in non-increasing key-tile count."""
    chunks = [(1024, 1024), (300, 300), (2000, 700), (64, 64), (5, 5)]
    b = dev(synth_prefill(91, chunks, 16))
    T = b["q"].shape[0]
    pws = ops.prefill_workspace(T, DEV)
    ops.paged_attention_prefill_plan(b["token_seq"], b["token_kv_len"], b["block_tables"].shape[1], 16, pws)
    torch.cuda.synchronize()
    G = (T + 63) // 64
    w = pws.cpu().numpy()
    order = w[G:2 * G]
    assert sorted(order.tolist()) == list(range(G))
    kvl, sq = b["token_kv_len"].cpu().numpy(), b["token_seq"].cpu().numpy()
    cost = [int(-(-max(kvl[g * 64:(g + 1) * 64][sq[g * 64:(g + 1) * 64] >= 0], default=0) // 32)) for g in range(G)]
    assert all(cost[order[i]] >= cost[order[i + 1]] for i in range(G - 1))


def test_prefill_kernel_rejects_unsupported_gqa():
    b = dev(synth_prefill(62, [(40, 8)], 16, H=12, KV=4))
    with pytest.raises(ops.CvhError if hasattr(ops, "CvhError") else Exception) as e:
        run_gpu(b, prefill=True)
    assert "UNSUPPORTED" in str(e.value)


@pytest.mark.parametrize("mode", PREFILL_MODES)
def test_prefill_kernel_ragged_edge_rows(orc, mode):
    say(f"prefill MFMA kernel: descending order, decode-like rows, kv_len 0 and padding rows, mode={mode}")
    b = synth_prefill(71, [(50, 50), (9, 1), (10, 1), (400, 3), (33, 33)], 16, order="desc")
    # a padding row (token_seq -1) and a zero-length row: all-zero outputs
    b["token_seq"][3] = -1
    b["token_kv_len"][7] = 0
    got = run_gpu(dev(b), prefill=mode)
    want = run_oracle(orc, b)
    assert not got[3].any() and not got[7].any()
    assert_close_bf16(got, want)


@pytest.mark.parametrize("mode", PREFILL_MODES)
def test_prefill_kernel_agrees_with_decode_kernel(mode):
    say(f"prefill MFMA kernel vs stream-K decode kernel on a 4096-token chunked batch, mode={mode}")
    chunks = [(1024, 1024), (2048, 1024), (3000, 1024), (600, 512), (900, 512)]
    b = dev(synth_prefill(81, chunks, 256))
    assert_close_bf16(run_gpu(b, prefill=mode), run_gpu(b), max_abs=1.6e-2, mean_abs=1e-3)


@pytest.mark.parametrize("tp", [2, 4, 8])
def test_tp_share_matches_full_heads(orc, tp):
    """One GPU's tensor-parallel shard of config 3 (kv heads [0, 8/tp), their query heads, the
    real contexts) gives the same output as those heads of the full 8-kv-head launch (within the
    tolerance: the work partition, and so the summation order, depends on the head count), and
    matches the oracle on a sample of its rows."""
    say(f"tp share {tp} of config 3 (64 sequences)")
    b = workloads.config3(device=DEV, seqs=64)
    full = run_gpu(b)
    s = workloads.tp_share(b, tp)
    shard = run_gpu(s)
    h = s["n_heads"]
    assert_close_bf16(shard, full[:, :h])
    rows = np.arange(0, 64, 9)
    assert_close_bf16(shard[rows], run_oracle(orc, s, rows))
