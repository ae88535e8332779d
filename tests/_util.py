"""Shared helpers for the parity tests: torch <-> numpy bit views and tolerance checks."""
import sys

import numpy as np
import torch

# The bar from the build's north star for bf16 attention / norm outputs.
MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def say(*a):
    """Name the case before a GPU step (and flush), so a crash log shows what ran."""
    print(*a, flush=True)
    sys.stdout.flush()


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor (any device) -> numpy uint16 bit patterns."""
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def f32_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().view(torch.int32).numpy().view(np.uint32)


def np_(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return bits(t)
    return t.detach().contiguous().cpu().numpy()


def bf16_vals(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_ulp(v: np.ndarray) -> np.ndarray:
    """Spacing of bf16 values at |v| (8 significant bits): 2^(floor(log2|v|) - 7)."""
    a = np.maximum(np.abs(np.asarray(v, np.float64)), 2.0 ** -126)
    return np.exp2(np.floor(np.log2(a)) - 7)


def assert_close_bf16(got_bits: np.ndarray, want_bits: np.ndarray, max_abs=MAX_ABS, mean_abs=MEAN_ABS,
                      ulp_floor=False):
    """max-abs / mean-abs bar on bf16 outputs. ulp_floor=True: an element may also differ by one
    bf16 ulp of the expected value where that ulp exceeds max_abs (|x| >= 4 for 2e-2). Two correct
    roundings of a value that sits near a bf16 rounding midpoint differ by one ulp, so outputs of
    large magnitude (config 4's 20x outliers) cannot meet an absolute 2e-2 bar."""
    g = bf16_vals(got_bits).astype(np.float64)
    w = bf16_vals(want_bits).astype(np.float64)
    assert np.isfinite(g).all(), "non-finite output"
    err = np.abs(g - w)
    tol = np.maximum(max_abs, bf16_ulp(w)) if ulp_floor else max_abs
    bad = err > tol
    assert not bad.any(), f"max-abs {err.max():.3e} > {max_abs}" + (
        f" and one ulp at {np.argwhere(bad)[0].tolist()}" if ulp_floor else "")
    assert err.mean() <= mean_abs, f"mean-abs {err.mean():.3e} > {mean_abs}"
    return float(err.max()), float(err.mean())


def to_dev(d: dict, device="cuda") -> dict:
    return {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in d.items()}
