"""GPU tests of the projections with fused epilogues (cvh_gemm_bf16_nt_residual,
cvh_gemm_bf16_nt_swiglu_rownorm, cvh_gemm_qkv_norm_rope_kv_write_fp8), through the C ABI.

* Residual epilogue: the new residual equals bf16(resid + y) with y the plain GEMM of the same
  tiled configuration (same fp32 sum order), bit for bit, and the per-16-column sums of squares
  equal their float32 restatement in the documented order, bit for bit.
* QKV epilogue without a row norm: q and every cache byte and scale equal the plain GEMM followed
  by the standalone QK-norm / RoPE / FP8-write kernel (itself bit-exact against the CPU oracle in
  test_gpu_fused.py), bit for bit, for every compiled tile, both scale modes and -1 slots.
* Row-normed consumers (x = raw residual, RMS factor from the partials, gain folded into the
  weight): within bf16 rounding of a float64 restatement of rnd(inv * x . w'^T); and the whole
  chain residual -> rownorm agrees with the unfused add_rms_norm + GEMM within the bar."""
import numpy as np
import pytest
import torch

from cppvllm_amd import _lib, ops
from tests._util import bf16_ulp, bf16_vals, bits, f32_bits, say

pytestmark = pytest.mark.gpu
DEV = "cuda"
TILED_PLAIN = 322222          # a tiled cvh_gemm_bf16_nt configuration (same sum order as every tiled one)


def codes(kind):
    L = _lib.lib()
    n = L.cvh_gemm_fused_configs(kind, None, 0)
    import ctypes as C
    buf = (C.c_int * n)()
    L.cvh_gemm_fused_configs(kind, buf, n)
    return list(buf)


def rnd(g, *shape, std=1.0):
    return (torch.randn(shape, generator=g) * std).to(torch.bfloat16)


def ss_restated(v_bits: np.ndarray) -> np.ndarray:
    """Per 16 columns: 4 lanes sum their 4 columns' squares in order (float32), then (s0+s1)+(s2+s3)."""
    v = bf16_vals(v_bits).astype(np.float32)
    M, N = v.shape
    q = v.reshape(M, N // 16, 4, 4)
    s = np.zeros((M, N // 16, 4), np.float32)
    with np.errstate(over="ignore"):               # rows of huge values overflow to inf, as on the GPU
        for r in range(4):
            s = (s + q[..., r] * q[..., r]).astype(np.float32)
        return ((s[..., 0] + s[..., 1]).astype(np.float32) + (s[..., 2] + s[..., 3]).astype(np.float32)).astype(
            np.float32)


def inv_restated(ss: np.ndarray, K: int, eps: float) -> np.ndarray:
    """Row factor from the partials: 4 lanes sum K/64 consecutive partials in order, then
    (q0+q1)+(q2+q3); inv = 1 / sqrt(sum / K + eps) in float32."""
    M = ss.shape[0]
    q = ss.reshape(M, 4, K // 64).astype(np.float32)
    acc = np.zeros((M, 4), np.float32)
    for i in range(K // 64):
        acc = (acc + q[:, :, i]).astype(np.float32)
    tot = ((acc[:, 0] + acc[:, 1]).astype(np.float32) + (acc[:, 2] + acc[:, 3]).astype(np.float32)).astype(np.float32)
    return (np.float32(1.0) / np.sqrt((tot / np.float32(K)).astype(np.float32) + np.float32(eps))).astype(np.float32)


@pytest.mark.parametrize("K", [2048, 3072])
@pytest.mark.parametrize("M", [1, 7, 64, 200, 256])
def test_residual_epilogue_bitexact(M, K):
    N = 1024
    g = torch.Generator().manual_seed(M * 7 + K)
    x, w, r0 = rnd(g, M, K), rnd(g, N, K, std=0.02), rnd(g, M, N)
    xd, wd = x.to(DEV), w.to(DEV)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    ops.linear(y, xd, wd, TILED_PLAIN if N % 64 == 0 else 0)
    want = (r0.to(DEV).float() + y.float()).to(torch.bfloat16)
    want_ss = ss_restated(bits(want))
    for c in codes(ops.FUSED_RESIDUAL) + [0]:
        say(f"residual epilogue M={M} N={N} K={K} config={c}")
        resid = r0.to(DEV)
        ss = torch.full((M, N // 16), float("nan"), device=DEV)
        ops.linear_residual(resid, ss, xd, wd, c)
        torch.cuda.synchronize()
        assert np.array_equal(bits(resid), bits(want)), f"config {c}"
        assert np.array_equal(f32_bits(ss), want_ss.view(np.uint32)), f"config {c}"


def _qkv_inputs(g, T, D, H, KV, HD, BS, NB, per_tensor):
    x = rnd(g, T, D)
    w = rnd(g, (H + 2 * KV) * HD, D, std=0.03)
    qn = (torch.rand((HD,), generator=g) + 0.5).to(torch.bfloat16)
    kn = (torch.rand((HD,), generator=g) + 0.5).to(torch.bfloat16)
    pos = torch.randint(0, 4000, (T,), generator=g)
    slots = torch.randperm(NB * BS, generator=g)[:T].clone()
    slots[::5] = -1                                       # padding rows: no cache writes
    cos, sin = ops.rope_tables(4096, HD, 1e6)
    if per_tensor:
        ks = torch.tensor([0.011]), torch.tensor([0.013])
    else:
        ks = torch.zeros((NB, KV, BS)), torch.zeros((NB, KV, BS))
    return x, w, qn, kn, pos, slots, cos, sin, ks


def _cache(NB, BS, KV, HD, scales):
    k = torch.full((NB, BS, KV, HD), 0xA5, dtype=torch.uint8, device=DEV)
    return k, k.clone(), scales[0].to(DEV).clone(), scales[1].to(DEV).clone()


@pytest.mark.parametrize("per_tensor", [False, True])
@pytest.mark.parametrize("T", [1, 5, 16, 33, 100, 256])
def test_qkv_epilogue_equals_gemm_then_kernel(T, per_tensor):
    D, H, KV, HD, BS, NB = 1024, 16, 8, 128, 16, 64
    g = torch.Generator().manual_seed(T * 3 + per_tensor)
    x, w, qn, kn, pos, slots, cos, sin, sc = _qkv_inputs(g, T, D, H, KV, HD, BS, NB, per_tensor)
    xd, wd, qnd, knd, posd, sld, cosd, sind = (t.to(DEV) for t in (x, w, qn, kn, pos, slots, cos, sin))
    qkv = torch.empty((T, (H + 2 * KV) * HD), dtype=torch.bfloat16, device=DEV)
    ops.linear(qkv, xd, wd, TILED_PLAIN)
    q_want = torch.empty((T, H, HD), dtype=torch.bfloat16, device=DEV)
    kw, vw, ksw, vsw = _cache(NB, BS, KV, HD, sc)
    ops.fused.qk_norm_rope_kv_write_fp8(q_want, qkv, qnd, knd, cosd, sind, posd, sld, kw, vw, ksw, vsw, None, None,
                                        H, KV, 1e-6)
    for c in codes(ops.FUSED_QKV) + [0]:
        say(f"qkv epilogue T={T} per_tensor={per_tensor} config={c}")
        q = torch.empty((T, H, HD), dtype=torch.bfloat16, device=DEV)
        kc, vc, ks, vs = _cache(NB, BS, KV, HD, sc)
        ops.qkv_norm_rope_kv_write_fp8(q, xd, None, 0.0, wd, qnd, knd, cosd, sind, posd, sld, kc, vc, ks, vs, H, KV,
                                       1e-6, c)
        torch.cuda.synchronize()
        assert np.array_equal(bits(q), bits(q_want)), f"config {c}"
        assert torch.equal(kc, kw) and torch.equal(vc, vw), f"config {c}"
        assert np.array_equal(f32_bits(ks), f32_bits(ksw)) and np.array_equal(f32_bits(vs), f32_bits(vsw))


def _rownorm_ref(v, ss, w_folded, eps):
    """float64 rnd(inv * v . w'^T) with inv from the restated partial sum."""
    K = v.size(1)
    inv = torch.from_numpy(inv_restated(ss.cpu().numpy(), K, eps)).double()
    return ((v.double().cpu() @ w_folded.double().cpu().T) * inv[:, None])


def _bar(got, want, what):
    """The north-star bar on bf16 outputs, plus: 99.5% of elements within two bf16 ulps of the
    reference (a gate/up value whose fp32 and float64 sums round to neighbouring bf16 values moves
    the product by about one ulp of each factor)."""
    g = got.double().cpu().numpy()
    w = want.double().cpu().numpy()
    err = np.abs(g - w)
    assert err.max() <= 2e-2 and err.mean() <= 2e-3, f"{what}: max {err.max():.3e} mean {err.mean():.3e}"
    near = (err <= 2 * bf16_ulp(w) + 1e-30).mean()
    assert near >= 0.995, f"{what}: only {near:.4f} within two ulps"


@pytest.mark.parametrize("M", [1, 24, 64, 130, 256])
def test_swiglu_rownorm(M):
    D, I, eps = 1024, 3072, 1e-6
    g = torch.Generator().manual_seed(M + 77)
    v = rnd(g, M, D)
    gain = (torch.rand((D,), generator=g) + 0.5).to(torch.bfloat16)
    wgu = rnd(g, 2 * I, D, std=0.02)
    wf = ops.fold_norm_gain(ops.interleave_gate_up(wgu), gain)
    ss = torch.from_numpy(ss_restated(bits(v)))
    # reference gate/up (interleaved order), then swiglu with the kernel's rounding points
    gu = _rownorm_ref(v, ss, wf, eps).to(torch.bfloat16)
    gu = gu.view(M, I // 16, 2, 16)
    gate, up = gu[:, :, 0, :].reshape(M, I), gu[:, :, 1, :].reshape(M, I)
    act_want = torch.empty((M, I), dtype=torch.bfloat16, device=DEV)
    ops.fused.swiglu(act_want, torch.cat([gate, up], 1).to(DEV))
    vd, ssd, wfd = v.to(DEV), ss.to(DEV), wf.to(DEV)
    for c in codes(ops.FUSED_SWIGLU_ROWNORM) + [0]:
        say(f"swiglu rownorm M={M} config={c}")
        act = torch.empty((M, I), dtype=torch.bfloat16, device=DEV)
        ops.linear_swiglu_rownorm(act, vd, ssd, eps, wfd, c)
        torch.cuda.synchronize()
        # a gate/up value one bf16 ulp off moves silu(g)*u by about one ulp of each factor
        _bar(act, act_want, f"config {c}")


@pytest.mark.parametrize("T", [3, 48, 256])
def test_qkv_rownorm_close_to_normed_path(T):
    """x = raw residual with row_ss: equals, within rounding, the unfused path that norms first."""
    D, H, KV, HD, BS, NB, eps = 1024, 16, 8, 128, 16, 64, 1e-6
    g = torch.Generator().manual_seed(T + 5)
    _, w, qn, kn, pos, slots, cos, sin, sc = _qkv_inputs(g, T, D, H, KV, HD, BS, NB, False)
    v = rnd(g, T, D)
    gain = (torch.rand((D,), generator=g) + 0.5).to(torch.bfloat16)
    ss = torch.from_numpy(ss_restated(bits(v)))
    qkv_ref = _rownorm_ref(v, ss, ops.fold_norm_gain(w, gain), eps).to(torch.bfloat16)
    d = lambda t: t.to(DEV)  # noqa: E731
    q_want = torch.empty((T, H, HD), dtype=torch.bfloat16, device=DEV)
    kw, vw, ksw, vsw = _cache(NB, BS, KV, HD, sc)
    ops.fused.qk_norm_rope_kv_write_fp8(q_want, d(qkv_ref), d(qn), d(kn), d(cos), d(sin), d(pos), d(slots), kw, vw,
                                        ksw, vsw, None, None, H, KV, eps)
    say(f"qkv rownorm T={T}")
    q = torch.empty((T, H, HD), dtype=torch.bfloat16, device=DEV)
    kc, vc, ks, vs = _cache(NB, BS, KV, HD, sc)
    ops.qkv_norm_rope_kv_write_fp8(q, d(v), d(ss), eps, d(ops.fold_norm_gain(w, gain)), d(qn), d(kn), d(cos), d(sin),
                                   d(pos), d(slots), kc, vc, ks, vs, H, KV, eps)
    torch.cuda.synchronize()
    err = (q.float() - q_want.float()).abs()
    assert err.max().item() < 0.05 and err.mean().item() < 2e-3, (err.max().item(), err.mean().item())
    # cache: dequantised K/V of written slots within a few e4m3 steps of the reference path
    w_rows = slots[slots >= 0]
    for got, want, gs, ws in ((kc, kw, ks, ksw), (vc, vw, vs, vsw)):
        gd = got.view(torch.float8_e4m3fn).float().view(NB * BS, KV, HD)[w_rows.to(DEV)]
        wd = want.view(torch.float8_e4m3fn).float().view(NB * BS, KV, HD)[w_rows.to(DEV)]
        gsc = gs.permute(0, 2, 1).reshape(NB * BS, KV)[w_rows.to(DEV)]
        wsc = ws.permute(0, 2, 1).reshape(NB * BS, KV)[w_rows.to(DEV)]
        e = (gd * gsc[..., None] - wd * wsc[..., None]).abs()
        assert e.max().item() < 0.15 and e.mean().item() < 0.01, (e.max().item(), e.mean().item())


@pytest.mark.parametrize("M", [5, 256])
def test_residual_then_rownorm_matches_add_rms_norm_path(M):
    """o_proj-style residual epilogue followed by a row-normed projection vs add_rms_norm + GEMM."""
    D, K, N, eps = 1024, 2048, 1024, 1e-6
    g = torch.Generator().manual_seed(M + 11)
    x, wo, h0 = rnd(g, M, K), rnd(g, D, K, std=0.02), rnd(g, M, D)
    gain = (torch.rand((D,), generator=g) + 0.5).to(torch.bfloat16)
    wn = rnd(g, N, D, std=0.03)
    d = lambda t: t.to(DEV)  # noqa: E731
    # unfused: y = x.wo^T; add_rms_norm(h, y, gain) -> normed; z = normed . wn^T
    h = d(h0)
    y = torch.empty((M, D), dtype=torch.bfloat16, device=DEV)
    ops.linear(y, d(x), d(wo), TILED_PLAIN)
    normed = torch.empty_like(y)
    ops.fused.add_rms_norm(h, y, d(gain), normed, eps)
    z_want = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    ops.linear(z_want, normed, d(wn))
    # fused: the residual epilogue, then the row factor from its partials (restated on the host)
    h2 = d(h0)
    ss = torch.empty((M, D // 16), device=DEV)
    ops.linear_residual(h2, ss, d(x), d(wo))
    torch.cuda.synchronize()
    say(f"residual -> rownorm chain M={M}")
    assert torch.equal(h2, h)
    z = _rownorm_ref(h2.cpu(), ss.cpu(), ops.fold_norm_gain(wn, gain), eps)
    # the two paths differ in where x is rounded: the fused one skips rounding the normed x
    # (twice) and so must be no further from the exact float64 result than the unfused one
    hv = h2.double().cpu()
    exact = ((hv * torch.rsqrt(hv.pow(2).mean(-1, keepdim=True) + eps)) * gain.double()) @ wn.double().T
    e_fused = (z.to(torch.bfloat16).double() - exact).abs()
    e_unfused = (z_want.double().cpu() - exact).abs()
    say(f"  vs exact: fused max {e_fused.max():.3e} mean {e_fused.mean():.3e}; "
        f"unfused max {e_unfused.max():.3e} mean {e_unfused.mean():.3e}")
    assert e_fused.max() <= 1.25 * e_unfused.max() and e_fused.mean() <= 1.25 * e_unfused.mean()


def _special_rows(g, M, D):
    """Residual rows whose sum of squares is zero, underflows (1e-25), is large but finite (1e15)
    or overflows to inf (1e19), among ordinary rows."""
    v = rnd(g, M, D).float()
    v[0] = 0.0
    v[1] *= 1e-25
    v[2] *= 1e15
    v[3] *= 1e19
    return v.to(torch.bfloat16)


def test_residual_epilogue_special_rows_bitexact():
    """The residual add and its partial sums of squares on rows of extreme magnitude (sums of
    squares that underflow to 0 or overflow to inf), bit for bit against the restatement."""
    M, N, K = 16, 1024, 2048
    g = torch.Generator().manual_seed(91)
    x, w, r0 = rnd(g, M, K), rnd(g, N, K, std=0.02), _special_rows(g, M, N)
    x[:2] = 0                    # rows 0, 1: the projection adds exact zeros, so the sums stay 0 / tiny
    xd, wd = x.to(DEV), w.to(DEV)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    ops.linear(y, xd, wd, TILED_PLAIN)
    want = (r0.to(DEV).float() + y.float()).to(torch.bfloat16)
    want_ss = ss_restated(bits(want))
    assert np.isinf(want_ss[3]).any() and (want_ss[0] == 0).all() and (want_ss[1] == 0).all()
    for c in codes(ops.FUSED_RESIDUAL) + [0]:
        say(f"residual epilogue special rows config={c}")
        resid = r0.to(DEV)
        ss = torch.full((M, N // 16), float("nan"), device=DEV)
        ops.linear_residual(resid, ss, xd, wd, c)
        torch.cuda.synchronize()
        assert np.array_equal(bits(resid), bits(want)), f"config {c}"
        assert np.array_equal(f32_bits(ss), want_ss.view(np.uint32)), f"config {c}"


def test_swiglu_rownorm_special_rows():
    """Row-normed gate/up on those rows: the row factor from the partials is 1/sqrt(eps) for a zero
    or underflowing sum and 0 for an overflowing one, as in the float64 restatement; outputs are
    finite and within the bar."""
    M, D, I, eps = 16, 1024, 3072, 1e-6
    g = torch.Generator().manual_seed(92)
    v = _special_rows(g, M, D)
    gain = (torch.rand((D,), generator=g) + 0.5).to(torch.bfloat16)
    wf = ops.fold_norm_gain(ops.interleave_gate_up(rnd(g, 2 * I, D, std=0.02)), gain)
    ss = torch.from_numpy(ss_restated(bits(v)))
    gu = _rownorm_ref(v, ss, wf, eps).to(torch.bfloat16).view(M, I // 16, 2, 16)
    gate, up = gu[:, :, 0, :].reshape(M, I), gu[:, :, 1, :].reshape(M, I)
    act_want = torch.empty((M, I), dtype=torch.bfloat16, device=DEV)
    ops.fused.swiglu(act_want, torch.cat([gate, up], 1).to(DEV))
    for c in codes(ops.FUSED_SWIGLU_ROWNORM) + [0]:
        say(f"swiglu rownorm special rows config={c}")
        act = torch.empty((M, I), dtype=torch.bfloat16, device=DEV)
        ops.linear_swiglu_rownorm(act, v.to(DEV), ss.to(DEV), eps, wf.to(DEV), c)
        torch.cuda.synchronize()
        assert torch.isfinite(act.float()).all(), f"config {c}"
        _bar(act, act_want, f"config {c}")
