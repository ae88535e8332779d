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


def assert_close_bf16(got_bits: np.ndarray, want_bits: np.ndarray, max_abs=MAX_ABS, mean_abs=MEAN_ABS):
    g = bf16_vals(got_bits).astype(np.float64)
    w = bf16_vals(want_bits).astype(np.float64)
    assert np.isfinite(g).all(), "non-finite output"
    err = np.abs(g - w)
    assert err.max() <= max_abs, f"max-abs {err.max():.3e} > {max_abs}"
    assert err.mean() <= mean_abs, f"mean-abs {err.mean():.3e} > {mean_abs}"
    return float(err.max()), float(err.mean())


def to_dev(d: dict, device="cuda") -> dict:
    return {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in d.items()}
