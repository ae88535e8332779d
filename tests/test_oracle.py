"""Pins the CPU oracle (oracle/cvh_oracle.c) against checks that do not reuse its code:
torch's own float8/bfloat16 casts, float64 recomputation, closed forms and invariants.
CPU only."""
import math

import numpy as np
import pytest
import torch

E4M3_MAX = 448.0


def torch_e4m3(x: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).clamp(-E4M3_MAX, E4M3_MAX)
    return t.to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def bf16_round64(x):
    """float64 -> nearest bf16 value (via float32 then torch's RNE cast)."""
    return torch.from_numpy(np.asarray(x, dtype=np.float32)).to(torch.bfloat16).float().numpy().astype(np.float64)


def to_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16)


# ---------------------------------------------------------------------------------------------- e4m3
def test_e4m3_encode_matches_torch_over_bit_patterns(orc):
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    lows = np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF, 0x4000, 0xC000], dtype=np.uint32)
    bits = (hi[:, None] | lows[None, :]).ravel()
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    got = orc.e4m3_quantize(x)
    want = torch_e4m3(x)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first x={x[bad[:5]]} got={got[bad[:5]]} want={want[bad[:5]]}"


def test_e4m3_encode_midpoints_and_boundaries(orc):
    table = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    pos = np.sort(table[(table >= 0) & np.isfinite(table)])
    mids = (pos[:-1].astype(np.float64) + pos[1:]) / 2
    cands = np.concatenate([pos, mids, np.nextafter(mids, 0), np.nextafter(mids, 1e9)]).astype(np.float32)
    cands = np.concatenate([cands, -cands])
    assert np.array_equal(orc.e4m3_quantize(cands), torch_e4m3(cands))
    # saturation and NaN closed forms
    sat = np.array([448, 449, 463.9, 464, 465, 480, 1e6, np.inf], dtype=np.float32)
    assert (orc.e4m3_quantize(sat) == 0x7E).all()
    assert (orc.e4m3_quantize(-sat) == 0xFE).all()
    assert orc.e4m3_quantize(np.array([np.nan], dtype=np.float32))[0] == 0x7F
    # subnormals k * 2^-9 and the smallest normal
    k = np.arange(0, 9, dtype=np.float32)
    assert np.array_equal(orc.e4m3_quantize(k * 2.0 ** -9), np.arange(0, 9, dtype=np.uint8))
    # ties to even at the bottom: 0.5 * 2^-9 -> 0, 1.5 * 2^-9 -> 2
    assert orc.e4m3_quantize(np.array([0.5 * 2 ** -9, 1.5 * 2 ** -9], dtype=np.float32)).tolist() == [0, 2]


def test_e4m3_decode_table(orc):
    got = orc.e4m3_decode_table()
    via_torch = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    finite = ~np.isnan(via_torch)
    assert np.isnan(got[0x7F]) and np.isnan(got[0xFF]) and finite.sum() == 254
    assert np.array_equal(got[finite], via_torch[finite])
    # spec formula, written independently: (-1)^s * 2^(e-7) * (1 + m/8), subnormal 2^-6 * m/8
    for c in range(256):
        s, e, m = c >> 7, (c >> 3) & 15, c & 7
        if e == 15 and m == 7:
            continue
        v = (m / 8) * 2.0 ** -6 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7)
        assert got[c] == (-v if s else v)


def test_bf16_rounding_matches_torch(orc):
    rng = np.random.default_rng(7)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-30, 30, 20000),
        # exact ties: bf16 value + half ulp
        ((rng.integers(0, 1 << 16, 4000).astype(np.uint32) << 16) | 0x8000).view(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38, -3.4e38, 1e-45], dtype=np.float32),
    ]).astype(np.float32)
    x = x[np.isfinite(x) | np.isinf(x)]
    got = orc.bf16_bits(x)
    want = to_bits(torch.from_numpy(x).to(torch.bfloat16))
    assert np.array_equal(got, want)


# ---------------------------------------------------------------------------------------------- norms
def _rand_bf16(shape, rng, scale=1.0):
    return to_bits(torch.from_numpy((rng.standard_normal(shape) * scale).astype(np.float32)).to(torch.bfloat16))


@pytest.mark.parametrize("D", [1024, 64, 136])
def test_rms_norm_vs_float64(orc, D):
    rng = np.random.default_rng(D)
    N = 64
    x = _rand_bf16((N, D), rng)
    w = to_bits(torch.from_numpy(rng.uniform(0.5, 1.5, D).astype(np.float32)).to(torch.bfloat16))
    eps = 1e-6
    got = orc.bf16_to_f32(orc.rms_norm(x, w, eps)).astype(np.float64)
    xv = orc.bf16_to_f32(x).astype(np.float64)
    wv = orc.bf16_to_f32(w).astype(np.float64)
    inv = 1.0 / np.sqrt((xv ** 2).sum(1, keepdims=True) / D + np.float32(eps))
    want = bf16_round64(bf16_round64(xv * inv) * wv)
    ulp = np.abs(want) * 2.0 ** -7 + 1e-30
    assert (np.abs(got - want) <= ulp).all()
    assert (got == want).mean() > 0.99


def test_rms_norm_constant_row_closed_form(orc):
    D = 1024
    c = 0.75
    x = np.full((1, D), 0x3F40, dtype=np.uint16)      # bf16(0.75)
    w = np.full(D, 0x3F80, dtype=np.uint16)           # bf16(1.0)
    out = orc.bf16_to_f32(orc.rms_norm(x, w, 1e-6))
    inv = np.float32(1.0) / np.sqrt(np.float32(c * c) + np.float32(1e-6), dtype=np.float32)
    want = bf16_round64(bf16_round64(np.float32(c) * inv))
    assert np.all(out == want)


def test_add_rms_norm_residual_exact_and_out(orc):
    rng = np.random.default_rng(3)
    N, D = 32, 1024
    r, x = _rand_bf16((N, D), rng), _rand_bf16((N, D), rng)
    w = to_bits(torch.from_numpy(rng.uniform(0.5, 1.5, D).astype(np.float32)).to(torch.bfloat16))
    new_r, out = orc.add_rms_norm(r, x, w, 1e-6)
    want_r = to_bits((from_bits(r).float() + from_bits(x).float()).to(torch.bfloat16))
    assert np.array_equal(new_r, want_r)
    assert np.array_equal(out, orc.rms_norm(new_r, w, 1e-6))


def test_rms_norm_f32_and_f16_dtypes(orc):
    rng = np.random.default_rng(11)
    x = rng.standard_normal((8, 256)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    out = orc.rms_norm(x, w, 1e-6, orc.F32).astype(np.float64)
    want = x / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6) * w
    assert np.abs(out - want).max() < 1e-5
    xh = x.astype(np.float16)
    wh = w.astype(np.float16)
    outh = orc.rms_norm(xh.view(np.uint16), wh.view(np.uint16), 1e-6, orc.F16).view(np.float16).astype(np.float64)
    wanth = xh.astype(np.float64) / np.sqrt((xh.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6) * wh
    assert np.abs(outh - wanth).max() < 4e-3 * np.abs(wanth).max()


# ------------------------------------------------------------------------------------- qk norm / rope
def rope_np(max_pos, hd, theta):
    inv = 1.0 / theta ** (np.arange(0, hd, 2, dtype=np.float64) / hd)
    ang = np.outer(np.arange(max_pos, dtype=np.float64), inv)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def _qkv_case(rng, T, H, KV, HD, BS, nb):
    qkv = _rand_bf16((T, (H + 2 * KV) * HD), rng)
    qn = to_bits(torch.from_numpy(rng.uniform(0.5, 1.5, HD).astype(np.float32)).to(torch.bfloat16))
    kn = to_bits(torch.from_numpy(rng.uniform(0.5, 1.5, HD).astype(np.float32)).to(torch.bfloat16))
    pos = rng.integers(0, 3000, T).astype(np.int64)
    slots = rng.permutation(nb * BS)[:T].astype(np.int64)
    slots[rng.random(T) < 0.1] = -1
    return qkv, qn, kn, pos, slots


@pytest.mark.parametrize("HD,BS", [(128, 256), (128, 16), (64, 32)])
def test_qk_norm_rope_kv_write_vs_float64(orc, HD, BS):
    rng = np.random.default_rng(HD + BS)
    T, H, KV, nb = 48, 16, 8, 8
    qkv, qn, kn, pos, slots = _qkv_case(rng, T, H, KV, HD, BS, nb)
    cos, sin = rope_np(3000, HD, 1e6)
    kc = np.full((nb, BS, KV, HD), 0xAA, dtype=np.uint8)
    vc = np.full((nb, BS, KV, HD), 0xAA, dtype=np.uint8)
    ks = np.full((nb, KV, BS), np.nan, dtype=np.float32)
    vs = np.full((nb, KV, BS), np.nan, dtype=np.float32)
    q_out, kd, vd = orc.qk_norm_rope_kv_write_fp8(qkv, qn, kn, cos, sin, pos, slots, kc, vc, ks, vs, H, KV, HD, BS,
                                                  dense=True)
    x = orc.bf16_to_f32(qkv).reshape(T, H + 2 * KV, HD).astype(np.float64)
    half = HD // 2

    def norm_rope(xh, w):
        inv = 1.0 / np.sqrt((xh ** 2).sum(-1, keepdims=True) / HD + np.float32(1e-6))
        n = bf16_round64(bf16_round64(xh * inv) * orc.bf16_to_f32(w).astype(np.float64))
        c = cos[pos][:, None, :].astype(np.float64)
        s = sin[pos][:, None, :].astype(np.float64)
        a, b = n[..., :half], n[..., half:]
        return np.concatenate([a * c - b * s, b * c + a * s], -1)

    q64 = norm_rope(x[:, :H], qn)
    qgot = orc.bf16_to_f32(q_out).astype(np.float64)
    qwant = bf16_round64(q64)
    assert (np.abs(qgot - qwant) <= np.abs(qwant) * 2.0 ** -7 + 1e-6).all()
    assert (qgot == qwant).mean() > 0.98
    k64 = bf16_round64(norm_rope(x[:, H:H + KV], kn))
    assert (np.abs(orc.bf16_to_f32(kd).astype(np.float64) - k64) <= np.abs(k64) * 2.0 ** -7 + 1e-6).all()
    assert np.array_equal(vd, qkv.reshape(T, H + 2 * KV, HD)[:, H + KV:])

    table = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    written = set()
    for t in range(T):
        s = int(slots[t])
        if s < 0:
            continue
        b, o = divmod(s, BS)
        written.add((b, o))
        for h in range(KV):
            # V: closed form, bit-exact (order-free amax, single IEEE ops, RNE encode)
            xv = x[t, H + KV + h].astype(np.float32)
            sc = np.float32(max(np.abs(xv).max(), np.float32(1e-8))) / np.float32(448.0)
            assert vs[b, h, o] == sc
            assert np.array_equal(vc[b, o, h], torch_e4m3(xv * (np.float32(1.0) / sc)))
            # K: scale from the float64 recomputation agrees within 2 ulp; bytes within one code
            ksc = np.float32(np.abs(k64[t, h]).max()) / np.float32(448)
            assert abs(float(ks[b, h, o]) - float(ksc)) <= 2 * np.spacing(ksc)
            dec = table[kc[b, o, h]] * ks[b, h, o]
            assert np.all(np.abs(dec - k64[t, h]) <= np.abs(k64[t, h]) * 2.0 ** -3 + 1e-3 * ksc)
    for b in range(nb):
        for o in range(BS):
            if (b, o) not in written:
                assert (kc[b, o] == 0xAA).all() and (vc[b, o] == 0xAA).all()
                assert np.isnan(ks[b, :, o]).all() and np.isnan(vs[b, :, o]).all()


def test_qk_norm_special_cases(orc):
    H, KV, HD, BS, nb = 2, 1, 128, 16, 1
    T = 2
    qkv = np.zeros((T, (H + 2 * KV) * HD), dtype=np.uint16)
    rng = np.random.default_rng(0)
    qkv[0] = _rand_bf16(((H + 2 * KV) * HD,), rng)          # token 0: random, pos 0
    pos = np.array([0, 5], dtype=np.int64)                  # token 1: all zeros
    slots = np.array([3, 7], dtype=np.int64)
    w = np.full(HD, 0x3F80, dtype=np.uint16)
    cos, sin = rope_np(8, HD, 1e6)
    kc = np.zeros((nb, BS, KV, HD), np.uint8)
    vc = np.zeros_like(kc)
    ks = np.zeros((nb, KV, BS), np.float32)
    vs = np.zeros_like(ks)
    q_out, _, _ = orc.qk_norm_rope_kv_write_fp8(qkv, w, w, cos, sin, pos, slots, kc, vc, ks, vs, H, KV, HD, BS)
    # pos 0: RoPE is the identity, so q = bf16(bf16(x*inv)*1)
    x0 = orc.bf16_to_f32(qkv[0, :HD])
    assert np.array_equal(q_out[0, 0], orc.rms_norm(qkv[0:1, :HD], w, 1e-6)[0])
    assert np.abs(orc.bf16_to_f32(q_out[0, 0]) - x0 / np.sqrt((x0.astype(np.float64) ** 2).mean() + 1e-6)).max() < 0.02
    # zero head: scale = 1e-8/448, all-zero bytes, q = 0
    assert ks[0, 0, 7] == np.float32(1e-8) / np.float32(448) and vs[0, 0, 7] == ks[0, 0, 7]
    # (RoPE can produce -0.0 = 0x80 from 0*cos with cos < 0: still an exact zero)
    assert ((kc[0, 7] & 0x7F) == 0).all() and (vc[0, 7] == 0).all() and ((q_out[1] & 0x7FFF) == 0).all()


def test_qk_per_tensor_scale(orc):
    rng = np.random.default_rng(5)
    T, H, KV, HD, BS, nb = 8, 4, 2, 128, 16, 2
    qkv, qn, kn, pos, slots = _qkv_case(rng, T, H, KV, HD, BS, nb)
    slots[:] = np.arange(T)
    cos, sin = rope_np(3000, HD, 1e6)
    kc = np.zeros((nb, BS, KV, HD), np.uint8)
    vc = np.zeros_like(kc)
    ks = np.array([0.01], np.float32)
    vs = np.array([0.02], np.float32)
    orc.qk_norm_rope_kv_write_fp8(qkv, qn, kn, cos, sin, pos, slots, kc, vc, ks, vs, H, KV, HD, BS,
                                  scale_mode=orc.PER_TENSOR)
    assert ks[0] == np.float32(0.01) and vs[0] == np.float32(0.02)
    xv = orc.bf16_to_f32(qkv).reshape(T, H + 2 * KV, HD)[:, H + KV:]
    want = torch_e4m3(xv * (np.float32(1) / np.float32(0.02)))
    assert np.array_equal(vc.reshape(-1, KV, HD)[:T], want)


# ------------------------------------------------------------------------------------------ attention
def _attn_case(rng, S, H, KV, HD, BS, lens, per_tensor=False):
    nblk = [math.ceil(L / BS) for L in lens]
    nb = sum(nblk) + 2
    perm = rng.permutation(nb)
    W = max(nblk)
    table = np.full((S, W), -1, np.int64)
    p = 0
    for i, n in enumerate(nblk):
        table[i, :n] = perm[p:p + n]
        p += n
    kc = rng.integers(0, 256, (nb, BS, KV, HD), dtype=np.uint8)
    vc = rng.integers(0, 256, (nb, BS, KV, HD), dtype=np.uint8)
    for c in (kc, vc):   # no NaN codes, keep magnitudes moderate (like quantised N(0,1) data)
        c[(c & 0x7F) == 0x7F] = 0x70
        c[(c & 0x7F) > 0x60] &= 0xDF
    if per_tensor:
        ks = np.array([0.01], np.float32)
        vs = np.array([0.02], np.float32)
    else:
        ks = rng.uniform(0.002, 0.02, (nb, KV, BS)).astype(np.float32)
        vs = rng.uniform(0.002, 0.02, (nb, KV, BS)).astype(np.float32)
    q = _rand_bf16((S, H, HD), rng)
    return q, kc, vc, ks, vs, table, np.arange(S, dtype=np.int64), np.array(lens, np.int64)


def attn_float64(q, kc, vc, ks, vs, table, tseq, tlen, H, KV, HD, BS, scale):
    dec = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).double().numpy()
    T = tlen.shape[0]
    out = np.zeros((T, H, HD))
    qf = (q.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    REP = H // KV
    for t in range(T):
        L = int(tlen[t])
        j = np.arange(L)
        slot = table[tseq[t], j // BS] * BS + j % BS
        b, o = slot // BS, slot % BS
        for g in range(KV):
            K = dec[kc[b, o, g]]
            V = dec[vc[b, o, g]]
            if ks.size == 1:
                kss, vss = np.full(L, float(ks[0])), np.full(L, float(vs[0]))
            else:
                kss, vss = ks[b, g, o].astype(np.float64), vs[b, g, o].astype(np.float64)
            for r in range(REP):
                h = g * REP + r
                s = (K @ qf[t, h]) * scale * kss
                p = np.exp(s - s.max())
                out[t, h] = (p * vss) @ V / p.sum()
    return out


@pytest.mark.parametrize("BS,HD,REP,per_tensor", [(16, 128, 2, False), (256, 128, 2, True), (32, 64, 4, False),
                                                 (64, 128, 1, False), (16, 128, 8, True)])
def test_attention_oracle_vs_float64(orc, BS, HD, REP, per_tensor):
    rng = np.random.default_rng(BS * HD + REP)
    KV = 2
    H = KV * REP
    lens = [1, 15, 16, 17, 33, 300, 700]
    S = len(lens)
    args = _attn_case(rng, S, H, KV, HD, BS, lens, per_tensor)
    scale = 1 / math.sqrt(HD)
    got = orc.bf16_to_f32(orc.paged_attention_fp8(*args, H, KV, HD, BS,
                                                  orc.PER_TENSOR if per_tensor else orc.PER_TOKEN_HEAD, scale))
    want = attn_float64(*args, H, KV, HD, BS, scale)
    err = np.abs(got - want)
    assert err.max() <= np.abs(want).max() * 2.0 ** -7 + 1e-6
    assert (err <= np.abs(want) * 2.0 ** -8 * 1.01 + 1e-7).mean() > 0.97


@pytest.mark.parametrize("tp", [2, 4, 8])
def test_tp_share_slices_heads(orc, tp):
    """workloads.tp_share (one GPU's shard under tensor parallelism over kv heads) keeps kv heads
    [0, 8/tp) of caches and scales and their query heads: the oracle on the shard equals the first
    16/tp heads of the oracle on the full batch, bit for bit (each (token, head) is computed
    independently)."""
    from cppvllm_amd import workloads
    b = workloads.decode_batch([40, 300, 17, 520], 16, 77)
    s = workloads.tp_share(b, tp)
    H, KV = b["n_heads"], b["n_kv_heads"]
    assert (s["n_heads"], s["n_kv_heads"]) == (H // tp, KV // tp)
    assert s["k_cache"].shape == (b["num_blocks"], 16, KV // tp, 128) and s["k_cache"].is_contiguous()

    def run(d):
        host = [d[k].numpy() if d[k].dtype != torch.bfloat16 else d[k].view(torch.int16).numpy().view(np.uint16)
                for k in ("q", "k_cache", "v_cache", "k_scale", "v_scale", "block_tables", "token_seq", "token_kv_len")]
        return orc.paged_attention_fp8(*host, d["n_heads"], d["n_kv_heads"], 128, 16, orc.PER_TOKEN_HEAD, d["scale"])
    full, shard = run(b), run(s)
    assert np.array_equal(shard, full[:, :H // tp])


def test_attention_known_answers(orc):
    rng = np.random.default_rng(1)
    H, KV, HD, BS = 2, 1, 128, 16
    q, kc, vc, ks, vs, table, tseq, _ = _attn_case(rng, 1, H, KV, HD, BS, [40])
    dec = orc.e4m3_decode_table()
    # kv_len = 1: out = bf16(vs0 * v0)
    out = orc.paged_attention_fp8(q, kc, vc, ks, vs, table, tseq, np.array([1], np.int64), H, KV, HD, BS)
    b0 = table[0, 0]
    want = orc.bf16_bits((dec[vc[b0, 0, 0]] * ks.dtype.type(vs[b0, 0, 0])).astype(np.float32))
    # compare values (acc starts at +0, so a -0 V element comes out as +0)
    assert np.array_equal(orc.bf16_to_f32(out[0, 0]), orc.bf16_to_f32(want))
    assert np.array_equal(orc.bf16_to_f32(out[0, 1]), orc.bf16_to_f32(want))
    # identical keys and scales: uniform softmax => mean of scaled V
    kc2 = kc.copy()
    kc2[:, :, 0] = kc[b0, 0, 0]
    ks2 = np.full_like(ks, 0.01)
    vs2 = np.full_like(vs, 0.01)
    out = orc.paged_attention_fp8(q, kc2, vc, ks2, vs2, table, tseq, np.array([40], np.int64), H, KV, HD, BS)
    j = np.arange(40)
    slot = table[0, j // BS] * BS + j % BS
    mean = (dec[vc[slot // BS, slot % BS, 0]].astype(np.float64) * 0.01).mean(0)
    assert np.abs(orc.bf16_to_f32(out[0, 0]) - mean).max() <= np.abs(mean).max() * 2 ** -7 + 1e-6
    # one dominant key: output equals that key's V row
    kc3 = np.zeros_like(kc)
    s7 = slot[7]
    kc3[s7 // BS, s7 % BS, 0] = 0x7E                 # 448 in every dimension
    q3 = np.full_like(q, 0x4000)                     # 2.0 everywhere
    out = orc.paged_attention_fp8(q3, kc3, vc, ks2, vs2, table, tseq, np.array([40], np.int64), H, KV, HD, BS)
    v7 = (dec[vc[s7 // BS, s7 % BS, 0]].astype(np.float32) * np.float32(0.01))
    assert np.abs(orc.bf16_to_f32(out[0, 0]) - v7).max() <= np.abs(v7).max() * 2 ** -7 + 1e-6


def test_attention_block_permutation_invariance(orc):
    rng = np.random.default_rng(9)
    H, KV, HD, BS = 4, 2, 128, 16
    lens = [50, 100, 3]
    q, kc, vc, ks, vs, table, tseq, tlen = _attn_case(rng, 3, H, KV, HD, BS, lens)
    base = orc.paged_attention_fp8(q, kc, vc, ks, vs, table, tseq, tlen, H, KV, HD, BS)
    nb = kc.shape[0]
    perm = rng.permutation(nb)                       # new physical id of old block b is perm[b]
    inv = np.argsort(perm)
    kc2, vc2 = kc[inv], vc[inv]
    ks2, vs2 = ks[inv], vs[inv]
    table2 = np.where(table >= 0, perm[np.maximum(table, 0)], -1)
    out = orc.paged_attention_fp8(q, kc2, vc2, ks2, vs2, table2, tseq, tlen, H, KV, HD, BS)
    assert np.array_equal(out, base)


# ------------------------------------------------------------------------------------------- metadata
def test_token_metadata_closed_form(orc):
    rng = np.random.default_rng(2)
    BS, S, W = 16, 5, 6
    q_lens = [3, 1, 0, 7, 2]
    cached = [10, 0, 4, 30, 60]
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int64)
    T = int(cu[-1]) + 3                              # 3 padding rows
    positions = np.zeros(T, np.int64)
    for j in range(S):
        positions[cu[j]:cu[j + 1]] = cached[j] + np.arange(q_lens[j])
    table = rng.permutation(S * W).reshape(S, W).astype(np.int64)
    table[4, 4:] = -1
    seq, slot, kvl = orc.token_metadata(cu, positions, table, BS)
    want_seq = np.searchsorted(cu[1:], np.arange(T), side="right")
    for t in range(T):
        if want_seq[t] >= S:
            assert (seq[t], slot[t], kvl[t]) == (-1, -1, 0)
            continue
        p = positions[t]
        assert seq[t] == want_seq[t]
        assert slot[t] == table[want_seq[t], p // BS] * BS + p % BS
        assert kvl[t] == p + 1


def test_rope_table_host_matches_numpy():
    from cppvllm_amd.ops import rope_tables
    cos, sin = rope_tables(4096, 128, 1e6)
    c, s = rope_np(4096, 128, 1e6)
    assert np.abs(cos.numpy() - c).max() <= 1.2e-7 and np.abs(sin.numpy() - s).max() <= 1.2e-7
    assert (cos.numpy() == c).mean() > 0.999
