"""GPU tests of the decode-projection GEMM (cvh_gemm_bf16_nt): every compiled configuration and
the automatic dispatch against a float64 reference of the same bf16 inputs, determinism, graph
replay and the error paths, through the C ABI."""
import ctypes as C

import pytest
import torch

from cppvllm_amd import _lib, ops
from tests._util import say

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _codes(fn="cvh_gemm_bf16_nt_configs"):
    f = getattr(_lib.lib(), fn)
    n = f(None, 0)
    buf = (C.c_int * n)()
    f(buf, n)
    return list(buf)


def _decode(code):
    """(kind, bn, k_unit, k_exact): output-tile width, the K granularity and, for one-shot
    kernels, the only K they take."""
    if code >= 100000:                       # tiled
        nf, wn = (code // 100) % 10, code % 10
        return "tiled", 16 * nf * wn, 128, None
    if code >= 10000:                        # one-shot
        nc, nwn = (code // 100) % 100, code % 10
        return "oneshot", 16 * nwn, None, (4 // nwn) * nc * 128
    nwn = code % 10
    return "stream", 16 * nwn, (4 // nwn) * 128, None


def _check(y, x, w):
    """Element-wise: |y - ref| <= 2^-8 |ref| (bf16 output rounding) + 2^-18 sum_k |x_k w_k|
    (fp32 accumulation in any order)."""
    xf = x.cpu().double()
    wf = w.cpu().double()
    ref = xf @ wf.t()
    mag = xf.abs() @ wf.abs().t()
    got = y.cpu().double()
    assert torch.isfinite(got).all()
    err = (got - ref).abs()
    tol = ref.abs() * 2.0**-8 + mag * 2.0**-18
    bad = (err > tol).nonzero()
    assert bad.numel() == 0, f"{bad.shape[0]} elements off, first {bad[:4].tolist()} err {err.max().item():.3g}"


def _inputs(M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16)
    w = (torch.randn((N, K), generator=g) * 0.05).to(torch.bfloat16)
    return x, w


@pytest.mark.parametrize("code", _codes())
def test_every_configuration(code):
    kind, bn, k_unit, k_exact = _decode(code)
    N = max(bn, 64) * 2
    # tiled: fewer and more 128-k chunks than LDS stages; streaming: one chunk per wave and several
    Ks = [k_exact] if k_exact else ([384, 1152] if kind == "tiled" else [k_unit, 4 * k_unit])
    for K in Ks:
        for M in (1, 19, 70):
            say(f"gemm config {code} ({kind}) M={M} N={N} K={K}")
            x, w = _inputs(M, N, K, code + M + K)
            y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV)
            ops.linear(y, x.to(DEV), w.to(DEV), code)
            torch.cuda.synchronize()
            _check(y, x, w)


QWEN = {"qkv": (4096, 1024), "o_proj": (1024, 2048), "gate_up": (6144, 1024), "down": (1024, 3072)}


@pytest.mark.parametrize("name", list(QWEN))
def test_auto_dispatch_qwen_shapes(name):
    N, K = QWEN[name]
    for M in (1, 9, 16, 33, 64, 100, 200, 256):
        say(f"gemm auto {name} M={M}")
        x, w = _inputs(M, N, K, M * 31 + N)
        y = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
        ops.linear(y, x.to(DEV), w.to(DEV))
        torch.cuda.synchronize()
        _check(y, x, w)


@pytest.mark.parametrize("code", [0] + _codes("cvh_gemm_bf16_nt_swiglu_configs"))
def test_swiglu_epilogue_bitexact(code):
    """Fused gate/up GEMM + SwiGLU == the same tiled GEMM, de-interleaved, then cvh_swiglu."""
    I, K = 512, 384
    for M in (1, 37, 130):
        say(f"gemm swiglu config {code} M={M} I={I} K={K}")
        x, w = _inputs(M, 2 * I, K, code + M)
        x = (x.float() * 2).to(torch.bfloat16)                 # gate values well into silu's curve
        wi = ops.interleave_gate_up(w).to(DEV)
        xd = x.to(DEV)
        act = torch.empty((M, I), dtype=torch.bfloat16, device=DEV)
        ops.linear_swiglu(act, xd, wi, code)
        plain = code if code else _lib.lib().cvh_gemm_bf16_nt_swiglu_config(M, I, K)
        gu_il = torch.empty((M, 2 * I), dtype=torch.bfloat16, device=DEV)
        ops.linear(gu_il, xd, wi, plain)
        gu = ops.deinterleave_gate_up(gu_il.t().contiguous()).t().contiguous()
        want = torch.empty_like(act)
        ops.fused.swiglu(want, gu)
        torch.cuda.synchronize()
        assert torch.equal(act.view(torch.int16), want.view(torch.int16))
        _check(gu, x, w)


def test_lm_head_shape():
    say("gemm auto lm_head M=3 N=151936")
    x, w = _inputs(3, 151936, 1024, 5)
    y = torch.empty((3, 151936), dtype=torch.bfloat16, device=DEV)
    ops.linear(y, x.to(DEV), w.to(DEV))
    torch.cuda.synchronize()
    _check(y, x, w)


def test_deterministic_and_graph_replay():
    say("gemm determinism + graph replay")
    x, w = _inputs(48, 4096, 1024, 9)
    xd, wd = x.to(DEV), w.to(DEV)
    y0 = torch.empty((48, 4096), dtype=torch.bfloat16, device=DEV)
    ops.linear(y0, xd, wd)
    y1 = torch.empty_like(y0)
    ops.linear(y1, xd, wd)
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)
    yg = torch.empty_like(y0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            ops.linear(yg, xd, wd)
    torch.cuda.current_stream().wait_stream(s)
    for i in range(3):
        yg.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, y0), f"replay {i}"
        ops.linear(y1, xd, wd)               # eager work between replays
        torch.cuda.synchronize()


def test_error_paths():
    say("gemm error paths")
    L = _lib.lib()
    x = torch.zeros((4, 256), dtype=torch.bfloat16, device=DEV)
    w = torch.zeros((64, 256), dtype=torch.bfloat16, device=DEV)
    y = torch.zeros((4, 64), dtype=torch.bfloat16, device=DEV)
    s = torch.cuda.current_stream().cuda_stream
    assert L.cvh_gemm_bf16_nt(y.data_ptr(), x.data_ptr(), w.data_ptr(), 0, 64, 256, 0, s) == _lib.CVH_OK
    assert L.cvh_gemm_bf16_nt(y.data_ptr(), x.data_ptr(), w.data_ptr(), 4, 56, 256, 0, s) == _lib.CVH_ERR_UNSUPPORTED
    assert L.cvh_gemm_bf16_nt(y.data_ptr(), x.data_ptr(), w.data_ptr(), 4, 64, 200, 0, s) == _lib.CVH_ERR_UNSUPPORTED
    assert L.cvh_gemm_bf16_nt(y.data_ptr(), x.data_ptr(), w.data_ptr(), 4, 64, 256, 10211, s) == _lib.CVH_ERR_UNSUPPORTED
    assert L.cvh_gemm_bf16_nt(y.data_ptr(), x.data_ptr(), w.data_ptr(), 4, 64, 256, 77, s) == _lib.CVH_ERR_UNSUPPORTED
    assert L.cvh_gemm_bf16_nt(None, x.data_ptr(), w.data_ptr(), 4, 64, 256, 0, s) == _lib.CVH_ERR_INVALID_ARG
    assert L.cvh_gemm_bf16_nt(y.data_ptr(), x.data_ptr(), w.data_ptr(), -1, 64, 256, 0, s) == _lib.CVH_ERR_INVALID_ARG
    torch.cuda.synchronize()
    assert float(y.float().abs().sum()) == 0.0
