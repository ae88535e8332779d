"""GPU parity of the fused pre-attention ops against the CPU oracle (bit-exact), through the C ABI.

Covers BASELINE config 2 at full size (4096 packed tokens, 32 segments, -1 padding slots) and
variants: block size 16 (the reference's) and 256, head_dim 64, per-tensor scales, optional
dense K/V outputs, f16/f32 norm rows."""
import math

import numpy as np
import pytest
import torch

from cppvllm_amd import ops, workloads
from tests._util import bits, f32_bits, np_, say

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_config2_add_rms_norm_bitexact(orc):
    say("config2 add_rms_norm T=4096 D=1024")
    w = workloads.fused_batch(seed=1002, device="cpu")
    resid, x, g = w["resid"].to(DEV), w["x"].to(DEV), w["w"].to(DEV)
    out = torch.empty_like(x)
    ops.fused.add_rms_norm(resid, x, g, out, 1e-6)
    torch.cuda.synchronize()
    r_want, o_want = orc.add_rms_norm(np_(w["resid"]), np_(w["x"]), np_(w["w"]), 1e-6)
    assert np.array_equal(bits(resid), r_want)
    assert np.array_equal(bits(out), o_want)


@pytest.mark.parametrize("N,D", [(1, 1024), (5, 1024), (7, 64), (3, 136), (2, 4096), (9, 8192)])
def test_rms_norm_bitexact_shapes(orc, N, D):
    say(f"rms_norm N={N} D={D}")
    g = torch.Generator().manual_seed(N * 1000 + D)
    x = torch.randn((N, D), generator=g).to(torch.bfloat16)
    wt = (torch.rand((D,), generator=g) + 0.5).to(torch.bfloat16)
    xd, wd = x.to(DEV), wt.to(DEV)
    out = torch.empty_like(xd)
    ops.fused.rms_norm(out, xd, wd, 1e-6)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out), orc.rms_norm(np_(x), np_(wt), 1e-6))


def test_norm_special_rows_bitexact(orc):
    """rms_norm / add_rms_norm on rows at the edges of fp32 sum-of-squares arithmetic, bit-exact:
    zeros (eps only), 1e-20 (squares underflow), 1e19 (the sum overflows to inf: the row maps to
    zero), a single huge element among ordinary ones, and bf16's largest finite value."""
    say("rms_norm special rows")
    g = torch.Generator().manual_seed(99)
    D = 1024
    x = torch.randn((8, D), generator=g)
    x[0] = 0.0
    x[1] *= 1e-20
    x[2] = 1e19
    x[3, 17] = 1e18
    x[4] = 3.38e38
    x[5, ::2] = 0.0
    xb = x.to(torch.bfloat16)
    wt = (torch.rand((D,), generator=g) + 0.5).to(torch.bfloat16)
    out = torch.empty((8, D), dtype=torch.bfloat16, device=DEV)
    ops.fused.rms_norm(out, xb.to(DEV), wt.to(DEV), 1e-6)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out), orc.rms_norm(np_(xb), np_(wt), 1e-6))
    r = torch.randn((8, D), generator=g).to(torch.bfloat16)
    rd = r.to(DEV)
    out2 = torch.empty_like(out)
    ops.fused.add_rms_norm(rd, xb.to(DEV), wt.to(DEV), out2, 1e-6)
    torch.cuda.synchronize()
    r_want, o_want = orc.add_rms_norm(np_(r), np_(xb), np_(wt), 1e-6)
    assert np.array_equal(bits(rd), r_want)
    assert np.array_equal(bits(out2), o_want)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_norm_other_dtypes_bitexact(orc, dtype):
    say(f"add_rms_norm dtype={dtype}")
    g = torch.Generator().manual_seed(5)
    r = torch.randn((33, 1024), generator=g).to(dtype)
    x = torch.randn((33, 1024), generator=g).to(dtype)
    wt = (torch.rand((1024,), generator=g) + 0.5).to(dtype)
    rd, xd, wd = r.to(DEV), x.to(DEV), wt.to(DEV)
    out = torch.empty_like(xd)
    ops.fused.add_rms_norm(rd, xd, wd, out, 1e-6)
    torch.cuda.synchronize()
    code = orc.F16 if dtype == torch.float16 else orc.F32
    view = (lambda t: t.numpy().view(np.uint16)) if dtype == torch.float16 else (lambda t: t.numpy())
    r_want, o_want = orc.add_rms_norm(view(r), view(x), view(wt), 1e-6, code)
    assert np.array_equal(view(rd.cpu()), r_want)
    assert np.array_equal(view(out.cpu()), o_want)


def _run_qkv(orc, w, HD, BS, per_tensor, dense, nb):
    H, KV = w["n_heads"], w["n_kv_heads"]
    T = w["positions"].shape[0]
    cos, sin = ops.rope_tables(int(w["max_position"]), HD, 1e6)
    kc = torch.full((nb, BS, KV, HD), 0xAA, dtype=torch.uint8)
    vc = kc.clone()
    if per_tensor:
        ks = torch.tensor([0.013], dtype=torch.float32)
        vs = torch.tensor([0.007], dtype=torch.float32)
    else:
        ks = torch.full((nb, KV, BS), float("nan"), dtype=torch.float32)
        vs = ks.clone()
    # device run
    q_out = torch.empty((T, H, HD), dtype=torch.bfloat16, device=DEV)
    dk = torch.empty((T, KV, HD), dtype=torch.bfloat16, device=DEV) if dense else None
    dv = torch.empty((T, KV, HD), dtype=torch.bfloat16, device=DEV) if dense else None
    kcd, vcd, ksd, vsd = kc.to(DEV), vc.to(DEV), ks.to(DEV), vs.to(DEV)
    ops.fused.qk_norm_rope_kv_write_fp8(q_out, w["qkv"].to(DEV), w["q_norm"].to(DEV), w["k_norm"].to(DEV),
                                        cos.to(DEV), sin.to(DEV), w["positions"].to(DEV), w["slots"].to(DEV), kcd,
                                        vcd, ksd, vsd, dk, dv, H, KV, 1e-6)
    torch.cuda.synchronize()
    # oracle run
    kco, vco, kso, vso = kc.numpy().copy(), vc.numpy().copy(), ks.numpy().copy(), vs.numpy().copy()
    q_want, kd_want, vd_want = orc.qk_norm_rope_kv_write_fp8(
        np_(w["qkv"]), np_(w["q_norm"]), np_(w["k_norm"]), cos.numpy(), sin.numpy(), w["positions"].numpy(),
        w["slots"].numpy(), kco, vco, kso, vso, H, KV, HD, BS, orc.PER_TENSOR if per_tensor else orc.PER_TOKEN_HEAD,
        1e-6, dense)
    assert np.array_equal(bits(q_out).reshape(q_want.shape), q_want)
    assert np.array_equal(kcd.cpu().numpy(), kco), "K cache bytes differ"
    assert np.array_equal(vcd.cpu().numpy(), vco), "V cache bytes differ"
    assert np.array_equal(f32_bits(ksd), kso.view(np.uint32)), "K scales differ"
    assert np.array_equal(f32_bits(vsd), vso.view(np.uint32)), "V scales differ"
    if dense:
        assert np.array_equal(bits(dk), kd_want) and np.array_equal(bits(dv), vd_want)


def test_config2_qk_norm_rope_kv_write_bitexact(orc):
    say("config2 qk_norm_rope_kv_write T=4096 BS=256 per-token")
    w = workloads.fused_batch(seed=1002, device="cpu")
    assert (w["slots"] < 0).any(), "config 2 must contain -1 padding slots"
    _run_qkv(orc, w, 128, 256, per_tensor=False, dense=False, nb=w["num_blocks"])


@pytest.mark.parametrize("BS,per_tensor,dense", [(16, False, True), (256, True, False), (32, False, False)])
def test_qk_norm_rope_kv_write_variants(orc, BS, per_tensor, dense):
    say(f"qk_norm_rope_kv_write T=512 BS={BS} per_tensor={per_tensor} dense={dense}")
    w = workloads.fused_batch(seed=77 + BS, device="cpu", T=512, n_segments=8, bs=BS)
    _run_qkv(orc, w, 128, BS, per_tensor, dense, nb=w["num_blocks"])


def test_qk_norm_rope_head_dim_64(orc):
    say("qk_norm_rope_kv_write HD=64")
    g = torch.Generator().manual_seed(64)
    T, H, KV, HD, BS = 100, 8, 2, 64, 16
    nb = math.ceil(T / BS) + 1
    w = {
        "n_heads": H, "n_kv_heads": KV, "max_position": 5000,
        "qkv": torch.randn((T, (H + 2 * KV) * HD), generator=g).to(torch.bfloat16),
        "q_norm": (torch.rand((HD,), generator=g) + 0.5).to(torch.bfloat16),
        "k_norm": (torch.rand((HD,), generator=g) + 0.5).to(torch.bfloat16),
        "positions": torch.randint(0, 5000, (T,), generator=g),
        "slots": torch.randperm(nb * BS, generator=g)[:T],
    }
    w["slots"][::7] = -1
    _run_qkv(orc, w, HD, BS, per_tensor=False, dense=True, nb=nb)


@pytest.mark.parametrize("per_tensor", [False, True])
def test_qk_norm_rope_kv_write_special_rows(orc, per_tensor):
    """Rows that exercise the edges of the scale and norm arithmetic, bit-exact against the oracle:
    an all-zero V head (amax 0: the 1e-8 scale floor), an all-zero K head (RMS of zeros: eps
    only), V at 1e4 and at 1e-30 (bf16 subnormal range), one V value near the bf16 maximum (every
    other code of the head flushes to zero), q at 1e-20, and with per-tensor scales V values far
    beyond 448 x scale (saturation to +-448)."""
    say(f"qk_norm_rope_kv_write special rows per_tensor={per_tensor}")
    g = torch.Generator().manual_seed(4242)
    T, H, KV, HD, BS = 64, 16, 8, 128, 16
    nb = math.ceil(T / BS) + 1
    qkv = torch.randn((T, (H + 2 * KV) * HD), generator=g)
    v0 = (H + KV) * HD                                   # first V column
    qkv[3, v0:v0 + HD] = 0.0                             # V head 0 of token 3: all zero
    qkv[7, H * HD:H * HD + HD] = 0.0                     # K head 0 of token 7: all zero
    qkv[5, v0:] *= 1e4
    qkv[6, v0:] *= 1e-30
    qkv[11, v0 + 5] = 3.0e38
    qkv[9, :H * HD] *= 1e-20
    qkv[13, v0:] *= 300.0                                # with per-tensor scale 0.007: |v| / s >> 448
    w = {
        "n_heads": H, "n_kv_heads": KV, "max_position": 40960,
        "qkv": qkv.to(torch.bfloat16),
        "q_norm": (torch.rand((HD,), generator=g) + 0.5).to(torch.bfloat16),
        "k_norm": (torch.rand((HD,), generator=g) + 0.5).to(torch.bfloat16),
        "positions": torch.randint(0, 40960, (T,), generator=g),
        "slots": torch.randperm(nb * BS, generator=g)[:T],
    }
    _run_qkv(orc, w, HD, BS, per_tensor=per_tensor, dense=True, nb=nb)


def test_fp8_quantize_matches_oracle(orc):
    say("fp8 quantize bit patterns")
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    x = (hi[:, None] | np.array([0, 0x7FFF, 0x8000, 0x8001], dtype=np.uint32)[None, :]).ravel().view(np.float32)
    xd = torch.from_numpy(x.copy()).to(DEV)
    out = torch.empty(x.shape, dtype=torch.uint8, device=DEV)
    ops.fp8_e4m3_quantize(out, xd, 1.0)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), orc.e4m3_quantize(x))


def test_token_metadata_matches_oracle(orc):
    say("token metadata")
    g = torch.Generator().manual_seed(3)
    S, W, BS = 40, 12, 16
    q_lens = torch.randint(0, 9, (S,), generator=g)
    cached = torch.randint(0, 100, (S,), generator=g)
    cu = torch.cat([torch.zeros(1, dtype=torch.int64), q_lens.cumsum(0)])
    T = int(cu[-1]) + 5
    pos = torch.zeros(T, dtype=torch.int64)
    for j in range(S):
        pos[cu[j]:cu[j + 1]] = cached[j] + torch.arange(int(q_lens[j]))
    table = torch.randperm(S * W, generator=g).view(S, W)
    table[3, 2:] = -1
    seq, slot, kvl = ops.build_token_metadata(cu.to(DEV), pos.to(DEV), table.to(DEV), BS)
    torch.cuda.synchronize()
    ws, wsl, wk = orc.token_metadata(cu.numpy(), pos.numpy(), table.numpy(), BS)
    assert np.array_equal(seq.cpu().numpy(), ws)
    assert np.array_equal(slot.cpu().numpy(), wsl)
    assert np.array_equal(kvl.cpu().numpy(), wk)


# (H, KV, HD) layouts, block sizes and row counts drawn per seed for the bit-exact sweep below
_QKV_LAYOUTS = [(16, 8, 128), (8, 8, 128), (32, 8, 128), (64, 8, 128), (8, 2, 64), (2, 1, 128), (4, 4, 64),
                (16, 4, 128)]


@pytest.mark.parametrize("seed", range(16))
def test_qk_norm_rope_kv_write_random_bitexact(orc, seed):
    """Seeded random layouts, block sizes 16-1024, 1-600 rows with random positions and slots (some
    -1), qkv magnitudes from 1e-3 to 30 (so the per-(token, head) scales span many binades), both
    scale modes, with and without the dense K/V outputs: q, cache bytes and scales bit-exact."""
    r = np.random.default_rng(seed)
    H, KV, HD = _QKV_LAYOUTS[r.integers(len(_QKV_LAYOUTS))]
    BS = int([16, 32, 64, 256, 1024][r.integers(5)])
    T = int(r.integers(1, 601))
    per_tensor, dense = bool(r.integers(2)), bool(r.integers(2))
    mag = float(10.0 ** r.uniform(-3, 1.5))
    say(f"qk_norm_rope_kv_write random seed={seed} H={H} KV={KV} HD={HD} BS={BS} T={T} per_tensor={per_tensor} "
        f"dense={dense} mag={mag:.3g}")
    g = torch.Generator().manual_seed(500 + seed)
    nb = math.ceil(T / BS) + 2
    w = {
        "n_heads": H, "n_kv_heads": KV, "max_position": 8192,
        "qkv": (torch.randn((T, (H + 2 * KV) * HD), generator=g) * mag).to(torch.bfloat16),
        "q_norm": (torch.rand((HD,), generator=g) + 0.5).to(torch.bfloat16),
        "k_norm": (torch.rand((HD,), generator=g) + 0.5).to(torch.bfloat16),
        "positions": torch.randint(0, 8192, (T,), generator=g),
        "slots": torch.randperm(nb * BS, generator=g)[:T],
    }
    w["slots"][torch.rand((T,), generator=g) < 0.1] = -1
    _run_qkv(orc, w, HD, BS, per_tensor, dense, nb=nb)
