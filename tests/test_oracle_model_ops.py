"""Pins the oracle's model ops (SwiGLU, Philox, sampler) with checks that do not reuse its code:
numpy float64 formulas with torch's rounding casts, published Philox known answers, numpy argmax."""
import numpy as np
import torch

from tests._util import bf16_vals


def _torch_bf16_bits(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).view(torch.int16) \
        .numpy().view(np.uint16)


def test_philox_known_answers(orc):
    # Random123 kat_vectors, philox4x32_10.
    kat = [
        ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
        ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
        ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
         [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
    ]
    for c, k, want in kat:
        assert list(orc.philox4x32_10(c, k)) == want


def test_swiglu_matches_float64_formula(orc):
    rng = np.random.default_rng(7)
    g = rng.standard_normal((37, 2 * 96)).astype(np.float32) * 4
    g[0, :8] = [0, -0.0, 30, -30, 100, -100, 1e-3, -1e-3]
    gu = _torch_bf16_bits(g)
    got = orc.swiglu(gu)
    x = bf16_vals(gu).astype(np.float64)
    gate, up = x[:, :96], x[:, 96:]
    with np.errstate(over="ignore"):
        silu = (gate / (1.0 + np.exp(-gate))).astype(np.float32)
    silu_b = bf16_vals(_torch_bf16_bits(silu)).astype(np.float32)
    want = _torch_bf16_bits(silu_b * up.astype(np.float32))
    assert np.array_equal(got, want)
    # closed forms: g = 0 -> 0; large positive g -> silu(g) = g; large negative -> 0
    o, u = bf16_vals(got[0]), bf16_vals(gu[0, 96:])
    assert o[0] == 0.0 and o[1] == 0.0
    assert o[2] == bf16_vals(_torch_bf16_bits(np.float32(30.0) * u[2]))
    assert o[4] == bf16_vals(_torch_bf16_bits(np.float32(100.0) * u[4]))
    assert abs(o[3]) < 1e-10 and abs(o[5]) < 1e-38


def test_swiglu_f32_rows(orc):
    rng = np.random.default_rng(8)
    gu = rng.standard_normal((5, 64)).astype(np.float32)
    got = orc.swiglu(gu, dtype=orc.F32)
    g, u = gu[:, :32].astype(np.float64), gu[:, 32:]
    silu = (g / (1.0 + np.exp(-g))).astype(np.float32)
    assert np.array_equal(got, silu * u)


def test_greedy_sampler_is_first_argmax(orc):
    rng = np.random.default_rng(9)
    V = 1000
    lg = rng.standard_normal((6, V)).astype(np.float32)
    lg[1, [5, 77, 999]] = 50.0                      # ties: the lowest index wins
    lg[2, :] = -np.inf
    lg[2, 123] = -1e30
    lg[3, 10] = np.nan                              # NaN never wins
    lg[0, :] = -np.inf                              # all -inf: index 0 (equal, lower index)
    got = orc.sample_tokens(lg)
    want = np.argmax(np.where(np.isnan(lg), -np.inf, lg), axis=1)
    assert list(got) == list(want)
    assert got[1] == 5
    # bf16 logits and a row subset
    b = _torch_bf16_bits(lg)
    rows = np.array([4, 0, 4], dtype=np.int64)
    assert list(orc.sample_tokens(b, rows=rows)) == list(np.argmax(bf16_vals(b)[rows], axis=1))


def test_gumbel_sampler_matches_closed_form(orc):
    rng = np.random.default_rng(10)
    V, R = 203, 4
    lg = rng.standard_normal((R, V)).astype(np.float32)
    temps = np.array([0.7, 1.0, 0.0, 2.5], dtype=np.float32)
    seed, offset = 0x1234_5678_9ABC_DEF0, 77
    got = orc.sample_tokens(lg, temps=temps, seed=seed, offset=offset)
    for r in range(R):
        if temps[r] <= 0:
            assert got[r] == np.argmax(lg[r])
            continue
        u = np.empty(V, dtype=np.float64)
        for j0 in range(0, V, 4):
            c = orc.philox4x32_10([j0 // 4, r, offset & 0xFFFFFFFF, offset >> 32],
                                  [seed & 0xFFFFFFFF, seed >> 32])
            for j in range(j0, min(j0 + 4, V)):
                u[j] = ((int(c[j - j0]) >> 8) + 0.5) / 16777216.0
        inv_t = np.float32(1.0) / np.float32(max(temps[r], 1e-5))
        score = (lg[r].astype(np.float64) * np.float64(inv_t) - np.log(np.maximum(-np.log(u), 1e-10))) \
            .astype(np.float32)
        assert got[r] == int(np.argmax(score))
    # same key -> same draw; another offset -> the stream changes
    assert list(orc.sample_tokens(lg, temps=temps, seed=seed, offset=offset)) == list(got)
    draws = {tuple(orc.sample_tokens(lg, temps=np.ones(R, np.float32), seed=1, offset=o)) for o in range(20)}
    assert len(draws) > 1
