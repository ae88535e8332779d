"""Attention outputs across V and K magnitudes, and with kv_len beyond the block table, against
the CPU oracle, through the C ABI.

The V scales (per (token, head) or per tensor) are multiplied by a factor f from 1e-6 to 3e5: the
codes stay the same, so V, and every output row, scale by exactly f in the oracle. Each entry
point (decode on VALU at GQA 2, decode on MFMA at GQA 8, the multi-query kernel plain and
planned) is checked on outputs divided by f at the build's bar (max-abs 2e-2, mean-abs 2e-3, one
bf16 ulp allowed), so a format whose range or precision depends on the magnitude of V (an fp16
product of softmax weight and V scale would overflow above ~1e5 and lose bits below ~1e-3) fails.
"""
import numpy as np
import pytest
import torch

from tests._util import bf16_vals, bf16_ulp, say
from tests.test_gpu_attention import dev, run_gpu, run_oracle, run_planned, synth, synth_prefill

pytestmark = pytest.mark.gpu

FACTORS = [1e-6, 1e-3, 1.0, 1e3, 3e5]


def _check_scaled(got_bits, want_bits, f):
    """The bar on outputs divided by f, compared on the unscaled values (where one-ulp
    differences are exact): |got - want| <= max(2e-2 f, one bf16 ulp of want); mean <= 2e-3 f."""
    g = bf16_vals(got_bits).astype(np.float64)
    w = bf16_vals(want_bits).astype(np.float64)
    assert np.isfinite(g).all(), "non-finite output"
    err = np.abs(g - w)
    tol = np.maximum(2e-2 * f, bf16_ulp(w))
    assert (err <= tol).all(), f"max-abs {err.max() / f:.3e} (scaled by 1/{f:g})"
    assert err.mean() <= 2e-3 * f, f"mean-abs {err.mean() / f:.3e} (scaled by 1/{f:g})"


def _scale_v(b, f):
    b = dict(b)
    b["v_scale"] = b["v_scale"] * f
    return b


@pytest.mark.parametrize("f", FACTORS)
@pytest.mark.parametrize("per_tensor", [False, True])
@pytest.mark.parametrize("H", [16, 64])
def test_decode_v_magnitudes(orc, f, per_tensor, H):
    say(f"decode V magnitude f={f:g} per_tensor={per_tensor} H={H}")
    b = _scale_v(synth(71, [40, 300, 1000, 17, 2500], 16, H=H, KV=8, per_tensor=per_tensor), f)
    want = run_oracle(orc, b)
    db = dev(b)
    got = run_gpu(db)
    _check_scaled(got, want, f)
    assert np.array_equal(run_planned(db), got)


@pytest.mark.parametrize("f", FACTORS)
@pytest.mark.parametrize("per_tensor", [False, True])
@pytest.mark.parametrize("mode", [True, "planned"])
def test_prefill_v_magnitudes(orc, f, per_tensor, mode):
    say(f"prefill V magnitude f={f:g} per_tensor={per_tensor} mode={mode}")
    b = _scale_v(synth_prefill(72, [(300, 300), (1000, 70), (40, 40)], 16, per_tensor=per_tensor), f)
    _check_scaled(run_gpu(dev(b), prefill=mode), run_oracle(orc, b), f)


@pytest.mark.parametrize("fk", [1e-4, 1e2, 1e4])
@pytest.mark.parametrize("per_tensor", [False, True])
def test_k_magnitudes_all_paths(orc, fk, per_tensor):
    """K scales multiplied by fk: the softmax goes from nearly uniform (1e-4) to one-hot (1e4,
    scores of ~1e5), together with V scaled by 1e3; decode (VALU and MFMA) and the multi-query
    kernel against the oracle at the bar (outputs divided by the V factor)."""
    say(f"K magnitude fk={fk:g} per_tensor={per_tensor}")
    for H in (16, 64):
        b = synth(73, [40, 300, 1000, 17, 2500], 16, H=H, KV=8, per_tensor=per_tensor)
        b = _scale_v(dict(b, k_scale=b["k_scale"] * fk), 1e3)
        want = run_oracle(orc, b)
        db = dev(b)
        got = run_gpu(db)
        _check_scaled(got, want, 1e3)
        assert np.array_equal(run_planned(db), got)
    b = synth_prefill(74, [(300, 300), (1000, 70), (40, 40)], 16, per_tensor=per_tensor)
    b = _scale_v(dict(b, k_scale=b["k_scale"] * fk), 1e3)
    want = run_oracle(orc, b)
    for mode in (True, "planned"):
        _check_scaled(run_gpu(dev(b), prefill=mode), want, 1e3)


@pytest.mark.parametrize("BS", [16, 256])
def test_kv_len_beyond_table_is_clamped(orc, BS):
    """token_kv_len larger than a row's block table holds (table_width x block_size) attends over the
    whole table, in every entry point as in the oracle (cvh_oracle.c clamps L the same way)."""
    say(f"kv_len beyond the table BS={BS}")
    b = synth(75, [40, 300, 1000, 17, 700], BS, queries_per_seq=3)
    W = b["block_tables"].shape[1]
    longest = int(np.argmax([40, 300, 1000, 17, 700]))
    rows = (b["token_seq"] == longest).nonzero().flatten()
    b["token_kv_len"][rows] = W * BS + 100 + torch.arange(rows.numel())
    want = run_oracle(orc, b)
    db = dev(b)
    got = run_gpu(db)
    _check_scaled(got, want, 1.0)
    assert np.array_equal(run_planned(db), got)
    for mode in (True, "planned"):
        _check_scaled(run_gpu(db, prefill=mode), want, 1.0)
