"""Pins the oracle's RMS-norm family and KV-cache writers with checks independent of its formulas:
a library RMS norm, complex-number rotation for the RoPE, hand-worked cache indices (including
the PA_NZ shapes of the reference's smoke test) and the unfused composition for the fused quant."""
import numpy as np
import torch

from oracle import golden as G

RNG = np.random.default_rng(1)


def test_add_rms_norm_matches_torch_rms_norm():
    x1 = RNG.standard_normal((7, 96)).astype(np.float32)
    x2 = RNG.standard_normal((7, 96)).astype(np.float32)
    g = RNG.uniform(0.5, 1.5, 96).astype(np.float32)
    y, rstd, x = G.add_rms_norm(x1, x2, g, 1e-6, "fp32")
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x1 + x2).double(), (96,), torch.from_numpy(g).double(),
                                       eps=1e-6)
    np.testing.assert_allclose(y, ref.numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(x, x1 + x2)
    assert rstd.shape == (7, 1)


def test_add_rms_norm_constant_row_closed_form():
    x1 = np.full((1, 64), 1.5, np.float32)
    x2 = np.full((1, 64), 0.5, np.float32)
    y, rstd, _ = G.add_rms_norm(x1, x2, np.ones(64, np.float32), 0.0, "fp32")
    assert rstd[0, 0] == np.float32(0.5)  # 1 / sqrt(2^2)
    assert (y == 1.0).all()


def test_add_rms_norm_bf16_outputs_are_rounded():
    x1 = RNG.standard_normal((3, 64)).astype(np.float32)
    y, _, x = G.add_rms_norm(x1, x1, np.ones(64, np.float32), 1e-6, "bf16")
    assert (G.round_bf16(y) == y).all() and (G.round_bf16(x) == x).all()


def test_fused_quant_equals_the_unfused_composition():
    # the fusion pattern (python/torchair/patterns/add_rms_norm_dynamic_quant.py:67-80) is exact
    x1 = RNG.standard_normal((9, 128)).astype(np.float32)
    x2 = RNG.standard_normal((9, 128)).astype(np.float32)
    g = RNG.uniform(0.5, 1.5, 128).astype(np.float32)
    sm = RNG.uniform(0.5, 2, 128).astype(np.float32)
    for dt in ("bf16", "fp16", "fp32"):
        y, _, x = G.add_rms_norm(x1, x2, g, 1e-6, dt)
        q_ref, s_ref = G.dynamic_quant(y, sm)
        y1, y2, xo, s1, s2 = G.add_rms_norm_dynamic_quant(x1, x2, g, sm, None, None, 1e-6, False, dt)
        assert (y1 == q_ref).all() and (s1 == s_ref).all() and (xo == x).all()
        assert y2 is None and s2 is None
    # beta shifts y before rounding; a second smooth scale gives an independent quantisation
    beta = RNG.standard_normal(128).astype(np.float32)
    sm2 = RNG.uniform(0.5, 2, 128).astype(np.float32)
    y1, y2, _, _, s2 = G.add_rms_norm_dynamic_quant(x1, x2, g, sm, sm2, beta, 1e-6, True, "bf16")
    y, _, _ = G.add_rms_norm(x1, x2, g, 1e-6, "fp32")
    yb = G.round_bf16((y + beta).astype(np.float32))
    assert (y2 == G.dynamic_quant(yb, sm2)[0]).all()


def test_interleave_rope_is_a_complex_rotation_of_pairs():
    d = 64
    x = RNG.standard_normal((5, d)).astype(np.float32)
    theta = RNG.uniform(-3, 3, (5, d // 2))
    cos = np.concatenate([np.cos(theta)] * 2, axis=-1).astype(np.float32)
    sin = np.concatenate([np.sin(theta)] * 2, axis=-1).astype(np.float32)
    out = G.interleave_rope(x, cos, sin)
    z = (x[:, 0::2].astype(np.float64) + 1j * x[:, 1::2]) * np.exp(1j * theta)
    np.testing.assert_allclose(out[:, :d // 2], z.real, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(out[:, d // 2:], z.imag, rtol=1e-5, atol=1e-5)
    # theta = 0 only de-interleaves
    np.testing.assert_array_equal(G.interleave_rope(x, np.ones_like(cos), np.zeros_like(sin)),
                                  np.concatenate([x[:, 0::2], x[:, 1::2]], axis=-1))


def test_scatter_norm_hand_case_and_negative_slots():
    key = np.arange(3 * 2 * 4, dtype=np.float32).reshape(3, 2, 4)
    kc = np.zeros((2, 4, 2, 4), np.float32)  # 2 blocks of 4 slots
    out, _ = G.scatter_pa_kv_cache(key, key, kc, kc, np.array([5, -1, 0]), "Norm")
    assert (out[1, 1] == key[0]).all()       # slot 5 = block 1, offset 1
    assert (out[0, 0] == key[2]).all()       # slot 0
    assert np.count_nonzero(out) == np.count_nonzero(key[0]) + np.count_nonzero(key[2])


def test_scatter_pa_nz_layout_of_the_reference_smoke_test():
    # tests/smoke/ge_test.py:244-267: bs 16 tokens, 4 heads, k 32 / v 64 dims, 2 blocks of 32, last dim 16
    t, h, dk, dv, nb, bsz, last = 16, 4, 32, 64, 2, 32, 16
    key = RNG.standard_normal((t, h, dk)).astype(np.float16).astype(np.float32)
    val = RNG.standard_normal((t, h, dv)).astype(np.float16).astype(np.float32)
    kc = RNG.standard_normal((nb, h * dk // last, bsz, last)).astype(np.float32)
    vc = np.zeros((nb, h * dv // last, bsz, last), np.float32)
    slots = RNG.choice(nb * bsz, t, replace=False)
    ko, vo = G.scatter_pa_kv_cache(key, val, kc, vc, slots, "PA_NZ")
    for i, s in enumerate(slots):
        blk, off = divmod(int(s), bsz)
        row_k = key[i].reshape(-1)
        for e in range(h * dk):  # element e of the token row: piece e // last, lane e % last
            assert ko[blk, e // last, off, e % last] == row_k[e]
        assert (vo[blk, :, off, :].reshape(-1) == val[i].reshape(-1)).all()
    untouched = np.ones(nb * bsz, bool)
    untouched[slots] = False
    for s in np.nonzero(untouched)[0]:
        blk, off = divmod(int(s), bsz)
        assert (ko[blk, :, off, :] == kc[blk, :, off, :]).all()


def _mla_inputs(b=2, s=3, dc=64, dr=16):
    kv = RNG.standard_normal((b, 1, s, dc + dr)).astype(np.float32)
    kv = G.round_bf16(kv)
    gamma = G.round_bf16(RNG.uniform(0.5, 1.5, dc).astype(np.float32))
    theta = RNG.uniform(-3, 3, (b, 1, s, dr // 2))
    cos = G.round_bf16(np.concatenate([np.cos(theta)] * 2, -1).astype(np.float32))
    sin = G.round_bf16(np.concatenate([np.sin(theta)] * 2, -1).astype(np.float32))
    return kv, gamma, cos, sin


def test_kv_rmsnorm_rope_cache_pa_matches_its_parts():
    b, s, dc, dr, nb, bsz = 2, 3, 64, 16, 3, 4
    kv, gamma, cos, sin = _mla_inputs(b, s, dc, dr)
    idx = np.array([0, 5, -1, 11, 2, 7])
    kc = np.zeros((nb, bsz, 1, dr), np.float32)
    cc = np.zeros((nb, bsz, 1, dc), np.float32)
    ko, co, kr, ckv = G.kv_rmsnorm_rope_cache(kv, gamma, cos, sin, idx, kc, cc, 1e-5, "PA")
    flat = kv.reshape(b * s, dc + dr)
    y, _, _ = G.add_rms_norm(flat[:, :dc], np.zeros_like(flat[:, :dc]), gamma, 1e-5, "bf16")
    np.testing.assert_array_equal(ckv.reshape(b * s, dc), y)
    rope = G.round_bf16(G.interleave_rope(flat[:, dc:], cos.reshape(b * s, dr), sin.reshape(b * s, dr)))
    np.testing.assert_array_equal(kr.reshape(b * s, dr), rope)
    for t, r in enumerate(idx):
        if r >= 0:
            assert (co.reshape(-1, dc)[r] == y[t]).all() and (ko.reshape(-1, dr)[r] == rope[t]).all()
    assert (co.reshape(-1, dc)[[1, 3, 4, 6, 8, 9, 10]] == 0).all()


def test_kv_rmsnorm_rope_cache_norm_layout_rows():
    b, s, dc, dr, scache = 2, 3, 32, 8, 5
    kv, gamma, cos, sin = _mla_inputs(b, s, dc, dr)
    pos = np.array([[4, 0, 2], [1, 3, -1]])
    kc = np.zeros((b, 1, scache, dr), np.float32)
    cc = np.zeros((b, 1, scache, dc), np.float32)
    ko, co, _, ckv = G.kv_rmsnorm_rope_cache(kv, gamma, cos, sin, pos, kc, cc, 1e-5, "Norm")
    for bi in range(b):
        for si in range(s):
            if pos[bi, si] >= 0:
                assert (co[bi, 0, pos[bi, si]] == ckv[bi, 0, si]).all()


def test_kv_rmsnorm_rope_cache_int8_latent_modes():
    b, s, dc, dr, nb, bsz = 1, 4, 64, 16, 2, 4
    kv, gamma, cos, sin = _mla_inputs(b, s, dc, dr)
    idx = np.array([6, 1, 3, 0])
    kc = np.zeros((nb, bsz, 1, dr), np.float32)
    cc = np.zeros((nb, bsz, 1, dc), np.int8)
    tok = np.zeros((nb, bsz), np.float32)
    _, co, _, ckv, ts = G.kv_rmsnorm_rope_cache(kv, gamma, cos, sin, idx, kc, cc, 1e-5, "PA", c_kv_token_scale=tok)
    q, sc = G.dynamic_quant(ckv.reshape(b * s, dc))
    for t, r in enumerate(idx):
        assert (co.reshape(-1, dc)[r] == q[t]).all() and ts.reshape(-1)[r] == sc[t]
    # static per-channel: round(v * scale + offset), clamped
    scale = np.full(dc, 20.0, np.float32)
    off = np.full(dc, 1.0, np.float32)
    _, co2, _, ckv2 = G.kv_rmsnorm_rope_cache(kv, gamma, cos, sin, idx, kc, cc, 1e-5, "PA", c_kv_scale=scale,
                                              c_kv_offset=off)
    want = np.clip(np.rint(ckv2.reshape(b * s, dc) * 20.0 + 1.0), -128, 127)
    np.testing.assert_array_equal(co2.reshape(-1, dc)[idx], want)


# ----------------------------------------------------------------------------- fused MoE grouped GEMMs
def _silu64(a):
    return a / (1.0 + np.exp(-a))


def test_grouped_matmul_swiglu_quant_brute_force():
    e, k, n = 3, 32, 8
    counts = np.array([2, 0, 3])
    m = 6  # one row past the grouped total
    x = RNG.integers(-127, 128, (m, k)).astype(np.int8)
    w = RNG.integers(-127, 128, (e, k, n)).astype(np.int8)
    ws = RNG.uniform(1e-3, 1e-2, (e, n)).astype(np.float32)
    xs = RNG.uniform(1e-3, 1e-2, m).astype(np.float32)
    y, s = G.grouped_matmul_swiglu_quant(x, w, ws, xs, counts, 1)
    ends = np.cumsum(counts)
    for r in range(m):
        g = int(np.searchsorted(ends, r, side="right"))
        if g >= e:
            assert s[r] == 0 and (y[r] == 0).all()
            continue
        d = (x[r].astype(np.int64) @ w[g].astype(np.int64)) * ws[g].astype(np.float64) * float(xs[r])
        h = _silu64(d[: n // 2]) * d[n // 2:]
        sc = np.abs(h).max() / 127
        assert abs(s[r] - sc) <= 1e-5 * sc
        assert np.abs(y[r].astype(int) - np.clip(np.rint(h / sc), -128, 127)).max() <= 1
    # cumulative group_list gives the same result
    y2, s2 = G.grouped_matmul_swiglu_quant(x, w, ws, xs, ends, 0)
    assert (y2 == y).all() and (s2 == s).all()


def test_grouped_matmul_finalize_routing_brute_force():
    e, k, n, t = 3, 16, 8, 4
    counts = np.array([3, 2, 3])
    m = int(counts.sum())
    x = RNG.integers(-127, 128, (m, k)).astype(np.int8)
    w = RNG.integers(-127, 128, (e, k, n)).astype(np.int8)
    sc = RNG.uniform(1e-3, 1e-2, (e, n)).astype(np.float32)
    pts = RNG.uniform(1e-3, 1e-2, m).astype(np.float32)
    logit = RNG.uniform(0, 1, m).astype(np.float32)
    row_index = np.array([2, 0, 3, 1, 0, 2, 3, 1])
    shared = RNG.standard_normal((2, n)).astype(np.float32)
    y = G.grouped_matmul_finalize_routing(x, w, counts, 1, sc, pts, None, logit, row_index, shared, 0.5, 1, t)
    want = np.zeros((t, n))
    g = np.repeat(np.arange(e), counts)
    for r in range(m):
        v = (x[r].astype(np.int64) @ w[g[r]].astype(np.int64)) * sc[g[r]].astype(np.float64) * float(pts[r])
        want[row_index[r]] += float(logit[r]) * v
    want[1:3] += 0.5 * shared
    np.testing.assert_allclose(y, want, rtol=1e-5, atol=1e-5)
