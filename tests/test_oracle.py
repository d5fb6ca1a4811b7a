"""Pins the CPU oracle with checks independent of its own formulas: closed forms, invariants,
brute force on tiny inputs and special cases that reduce to library routines."""
import itertools
import math

import numpy as np
import pytest
import scipy.special

from oracle import golden as G

RNG = np.random.default_rng(0)


# ----------------------------------------------------------------------------- quantisation
def test_dynamic_quant_closed_form_and_round_half_even():
    # scale = 127/127 = 1 exactly, so y = rint(x): halves go to the even neighbour.
    x = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.49]], np.float32)
    y, s = G.dynamic_quant(x)
    assert s[0] == 1.0
    assert y[0].tolist() == [127, 0, 2, 2, 0, -2, -2, 3]


def test_dynamic_quant_invariants():
    x = RNG.standard_normal((64, 333)).astype(np.float32)
    x[3] = 0.0
    x[5] = 2.0
    y, s = G.dynamic_quant(x)
    assert np.abs(y.astype(int)).max() <= 127
    nz = np.abs(x).max(axis=1) > 0
    assert (np.abs(y[nz].astype(int)).max(axis=1) == 127).all()
    assert s[3] == 0 and (y[3] == 0).all()
    assert (y[5] == 127).all()
    # dequantised value within half a step of the input (plus fp32 rounding slack)
    err = np.abs(y.astype(np.float64) * s[:, None] - x)
    assert (err <= s[:, None] * 0.5 * (1 + 1e-5) + 1e-12).all()


def test_dynamic_quant_smooth_is_prescaling():
    x = RNG.standard_normal((10, 32)).astype(np.float32)
    sm = RNG.uniform(0.5, 2, 32).astype(np.float32)
    y1, s1 = G.dynamic_quant(x, sm)
    y2, s2 = G.dynamic_quant(x * sm)
    assert (y1 == y2).all() and (s1 == s2).all()
    # grouped smooth scales: rows [0,3) use row 0, [3,10) row 1 (cumulative ends)
    sm2 = RNG.uniform(0.5, 2, (2, 32)).astype(np.float32)
    y3, _ = G.dynamic_quant(x, sm2, np.array([3, 10]))
    assert (y3[:3] == G.dynamic_quant(x[:3] * sm2[0])[0]).all()
    assert (y3[3:] == G.dynamic_quant(x[3:] * sm2[1])[0]).all()


def _silu64(a):
    return a / (1.0 + math.exp(-a))


def test_dequant_swiglu_quant_brute_force():
    x = RNG.integers(-3000, 3000, (4, 16)).astype(np.int32)
    ws = RNG.uniform(1e-3, 1e-2, 16).astype(np.float32)
    act = RNG.uniform(0.01, 0.1, 4).astype(np.float32)
    for left in (True, False):
        y, s = G.dequant_swiglu_quant(x, ws, act, activate_left=left)
        for r in range(4):
            vals = []
            for j in range(8):
                a = float(x[r, j]) * float(ws[j]) * float(act[r])
                b = float(x[r, 8 + j]) * float(ws[8 + j]) * float(act[r])
                vals.append(_silu64(a) * b if left else a * _silu64(b))
            sc = max(abs(v) for v in vals) / 127.0
            assert s[r] == pytest.approx(sc, rel=1e-5)
            want = [max(-128, min(127, round(v / sc))) for v in vals]
            assert np.abs(y[r].astype(int) - np.array(want)).max() <= 1


def test_dequant_swiglu_quant_groups_and_zero_half():
    x = RNG.integers(-1000, 1000, (6, 8)).astype(np.int32)
    x[:, :4] = 0  # A half zero: silu(A)*B == 0 -> zero rows when activating the left half
    ws = RNG.uniform(1e-3, 1e-2, (2, 8)).astype(np.float32)
    y, s = G.dequant_swiglu_quant(x, ws, None, group_index=np.array([2, 3]), activate_left=True)
    assert (y == 0).all() and (s == 0).all()
    y, s = G.dequant_swiglu_quant(x, ws, None, group_index=np.array([2, 3]), activate_left=False)
    assert (s[5] == 0) and (y[5] == 0).all()  # row past the grouped total
    assert s[0] == 0  # A*silu(B) with A == 0
    # rows 0-1 use weight row 0, rows 2-4 weight row 1
    x2 = RNG.integers(-1000, 1000, (5, 8)).astype(np.int32)
    y2, _ = G.dequant_swiglu_quant(x2, ws, None, group_index=np.array([2, 3]))
    assert (y2[:2] == G.dequant_swiglu_quant(x2[:2], ws[0])[0]).all()
    assert (y2[2:] == G.dequant_swiglu_quant(x2[2:], ws[1])[0]).all()


# ----------------------------------------------------------------------------- GEMMs
def test_int_matmul_exact_at_cfg_k():
    a = np.full((2, 7168), -127, np.int8)
    b = np.full((7168, 3), -127, np.int8)
    acc = G.int_matmul(a, b)
    assert (acc == 127 * 127 * 7168).all()
    a = RNG.integers(-127, 128, (9, 700), dtype=np.int8)
    b = RNG.integers(-127, 128, (700, 5), dtype=np.int8)
    assert (G.int_matmul(a, b) == a.astype(np.int64) @ b.astype(np.int64)).all()


def test_quant_matmul_identity_and_epilogue():
    a = RNG.integers(-127, 128, (8, 16), dtype=np.int8)
    eye = np.eye(16, dtype=np.int8)
    assert (G.quant_matmul(a, eye, out_dtype="int32") == a.astype(np.int32)).all()
    scale = RNG.uniform(1e-3, 1e-2, 16).astype(np.float32)
    pts = RNG.uniform(1e-3, 1e-2, 8).astype(np.float32)
    out = G.quant_matmul(a, eye, scale, pts, None, "fp32")
    np.testing.assert_allclose(out, a.astype(np.float64) * scale[None] * pts[:, None], rtol=1e-6)
    bf = G.quant_matmul(a, eye, scale, pts, None, "bf16")
    np.testing.assert_allclose(bf, out, rtol=2 ** -8)


def test_grouped_matmul_is_per_group_matmul():
    x = RNG.integers(-127, 128, (20, 12), dtype=np.int8)
    w = RNG.integers(-127, 128, (3, 12, 5), dtype=np.int8)
    counts = np.array([7, 0, 10])
    out = G.grouped_matmul(x, w, counts, 1)
    assert (out[:7] == x[:7].astype(int) @ w[0].astype(int)).all()
    assert (out[7:17] == x[7:17].astype(int) @ w[2].astype(int)).all()
    assert (out[17:] == 0).all()
    assert (G.grouped_matmul(x, w, np.cumsum(counts), 0) == out).all()


# ----------------------------------------------------------------------------- gating
def _gate_brute(x, bias, k, k_group, group_count, mode):
    """Brute force over every choice of k_group groups, plain Python."""
    e = len(x)
    s = [1.0 / (1.0 + math.exp(-v)) for v in x]
    sb = [s[i] + bias[i] for i in range(e)]
    gsz = e // group_count
    def gscore(gi):
        vals = sorted(sb[gi * gsz:(gi + 1) * gsz], reverse=True)
        return vals[0] + vals[1] if mode == 1 else vals[0]
    scores = [gscore(gi) for gi in range(group_count)]
    best = None
    for combo in itertools.combinations(range(group_count), k_group):
        key = (sorted([-scores[c] for c in combo]), combo)
        if best is None or key < best:
            best = key
    cand = [i for c in best[1] for i in range(c * gsz, (c + 1) * gsz)]
    chosen = sorted(cand, key=lambda i: (-sb[i], i))[:k]
    w = [s[i] for i in chosen]
    tot = sum(w)
    return chosen, [v / tot for v in w]


def test_gating_brute_force():
    for trial in range(20):
        x = RNG.standard_normal((1, 16)).astype(np.float32)
        bias = (RNG.standard_normal(16) * 0.1).astype(np.float32)
        y, idx, _ = G.moe_gating_top_k(x, 3, bias, k_group=2, group_count=4, group_select_mode=trial % 2,
                                       norm_type=1)
        want_idx, want_w = _gate_brute(x[0].astype(np.float64), bias.astype(np.float64), 3, 2, 4, trial % 2)
        assert idx[0].tolist() == want_idx
        np.testing.assert_allclose(y[0], want_w, rtol=1e-5)


def test_gating_single_group_is_topk_and_softmax():
    x = RNG.standard_normal((50, 40)).astype(np.float32)
    y, idx, out = G.moe_gating_top_k(x, 5, norm_type=0, out_flag=True)
    p = scipy.special.softmax(x.astype(np.float64), axis=1)
    np.testing.assert_allclose(out, p, rtol=1e-6)
    want = np.argsort(-p, axis=1, kind="stable")[:, :5]
    assert (idx == want).all()
    np.testing.assert_allclose(y, np.take_along_axis(p, want, 1), rtol=1e-6)


def test_gating_ties_lower_index():
    x = np.zeros((1, 16), np.float32)
    _, idx, _ = G.moe_gating_top_k(x, 4, k_group=2, group_count=4, group_select_mode=1, norm_type=1)
    assert idx[0].tolist() == [0, 1, 2, 3]


# ----------------------------------------------------------------------------- routing
def test_init_routing_v2_invariants_and_round_trip():
    t, k, e, h = 50, 4, 9, 6
    idx = np.stack([RNG.permutation(e)[:k] for _ in range(t)]).astype(np.int32)
    x = RNG.standard_normal((t, h)).astype(np.float32)
    ex, ri, tok, _ = G.moe_init_routing_v2(x, idx, None, t * k, 0, e, 0, 0)
    assert sorted(ri.tolist()) == list(range(t * k))  # bijection
    src = np.empty(t * k, np.int64)
    src[ri] = np.arange(t * k)
    exp_sorted = idx.reshape(-1)[src]
    assert (np.diff(exp_sorted) >= 0).all()  # sorted by expert
    same = np.diff(exp_sorted) == 0
    assert (np.diff(src)[same] > 0).all()  # stable: slot order inside an expert
    assert tok[-1] == t * k and (np.diff(tok) >= 0).all()
    assert (ex == x[src // k]).all()
    _, ri1, cnt, _ = G.moe_init_routing_v2(x, idx, None, t * k, 0, e, 1, 1)
    assert (ri1 == src).all() and (np.cumsum(cnt) == tok).all()
    w = np.full((t, k), 1.0 / k, np.float32)
    y = G.moe_finalize_routing(ex, None, None, None, w, ri, idx, 2, "fp32")
    np.testing.assert_allclose(y, x, rtol=1e-6, atol=1e-6)


def test_init_routing_legacy_declared_case():
    """Declared case of moe_init_routing.py:4-9: F32(3,4), I32(3,2), I32(3,2), active_num=3."""
    x = RNG.standard_normal((3, 4)).astype(np.float32)
    row = np.arange(6, dtype=np.int32).reshape(2, 3).T
    idx = np.array([[2, 0], [1, 2], [0, 1]], np.int32)
    ex, eri, eei = G.moe_init_routing(x, row, idx, 3)
    assert eei.tolist() == [0, 0, 1, 1, 2, 2]
    # slot order (t*k+j): (0,1)->row 3,(2,0)->row 2 for expert 0; (1,0)->1,(2,1)->5; (0,0)->0,(1,1)->4
    assert (ex == x[np.array([3, 2, 1, 5, 0, 4]) % 3]).all()
    assert sorted(eri.tolist()) == list(range(6))


def test_finalize_declared_case_by_hand():
    ex = RNG.standard_normal((24, 7)).astype(np.float32)
    s1 = RNG.standard_normal((12, 7)).astype(np.float32)
    bias = RNG.standard_normal((3, 7)).astype(np.float32)
    sc = RNG.standard_normal((12, 2)).astype(np.float32)
    row = np.arange(24, dtype=np.int32)
    exp = RNG.integers(0, 3, (12, 2)).astype(np.int32)
    y = G.moe_finalize_routing(ex, s1, None, bias, sc, row, exp, 0, "fp32")
    for t in range(12):
        want = s1[t].astype(np.float64).copy()
        for j in range(2):
            want += sc[t, j] * (ex[j * 12 + t] + bias[exp[t, j]])
        np.testing.assert_allclose(y[t], want, rtol=1e-5, atol=1e-5)


# ----------------------------------------------------------------------------- attention
def _paged(L_list, hkv, d, bs, rng):
    nblk = sum((L + bs - 1) // bs for L in L_list) + 2
    k = rng.standard_normal((nblk, bs, hkv, d)).astype(np.float32)
    v = rng.standard_normal((nblk, bs, hkv, d)).astype(np.float32)
    perm = rng.permutation(nblk)
    width = max((L + bs - 1) // bs for L in L_list)
    bt = np.zeros((len(L_list), width), np.int32)
    o = 0
    for b, L in enumerate(L_list):
        nb = (L + bs - 1) // bs
        bt[b, :nb] = perm[o:o + nb]
        o += nb
    return k, v, bt


def test_paged_decode_matches_dense_and_lse():
    L = [5, 17, 1]
    k, v, bt = _paged(L, 2, 8, 4, RNG)
    q = RNG.standard_normal((3, 4, 8)).astype(np.float32)
    out, lse = G.paged_decode_attention(q, k, v, bt, L, 0.3)
    for b in range(3):
        kk = k[bt[b]].reshape(-1, 2, 8)[:L[b]]
        vv = v[bt[b]].reshape(-1, 2, 8)[:L[b]]
        for h in range(4):
            s = kk[:, h // 2].astype(np.float64) @ q[b, h] * 0.3
            p = scipy.special.softmax(s)
            np.testing.assert_allclose(out[b, h], p @ vv[:, h // 2], rtol=1e-4, atol=1e-5)
            assert lse[b, h] == pytest.approx(scipy.special.logsumexp(s), rel=1e-5)
    # L == 1 -> the single value row
    np.testing.assert_allclose(out[2, 0], v[bt[2, 0], 0, 0], rtol=1e-6)


def test_paged_decode_constant_values():
    k, v, bt = _paged([9, 12], 1, 4, 4, RNG)
    v[:] = np.arange(4, dtype=np.float32)
    out, _ = G.paged_decode_attention(RNG.standard_normal((2, 3, 4)).astype(np.float32), k, v, bt, [9, 12], 1.0)
    np.testing.assert_allclose(out, np.broadcast_to(np.arange(4, dtype=np.float32), out.shape), rtol=1e-5)


def test_prefill_causal_prefix_property():
    q = RNG.standard_normal((1, 6, 2, 4)).astype(np.float32)
    k = RNG.standard_normal((1, 6, 1, 4)).astype(np.float32)
    v = RNG.standard_normal((1, 6, 1, 4)).astype(np.float32)
    out, _ = G.prefill_attention(q, k, v, None, None, 1, 0.5)
    k2, v2 = k.copy(), v.copy()
    k2[0, 4:] = 100.0
    v2[0, 4:] = -50.0
    out2, _ = G.prefill_attention(q, k2, v2, None, None, 1, 0.5)
    np.testing.assert_allclose(out[0, :4], out2[0, :4], rtol=1e-6)  # rows < 4 never see kv >= 4
    np.testing.assert_allclose(out[0, 0, 0], v[0, 0, 0], rtol=1e-6)  # first row sees only kv 0
    # padded query rows are zero
    out3, lse3 = G.prefill_attention(q, k, v, [3], [3], 1, 0.5)
    assert (out3[0, 3:] == 0).all() and np.isneginf(lse3[0, :, 3:]).all()


def test_band_mask_rules():
    big = 2147483647
    # the causal modes
    for lq, lk in ((5, 5), (3, 7), (6, 6)):
        ii, jj = np.arange(lq)[:, None], np.arange(lk)[None, :]
        np.testing.assert_array_equal(G.band_mask(lq, lk, 1, big, 0), jj <= ii + (lk - lq))
        np.testing.assert_array_equal(G.band_mask(lq, lk, 0, big, 0), jj <= ii)
        assert G.band_mask(lq, lk, 0, big, big).all() and G.band_mask(lq, lk, 1, big, big).all()
    # visible count per row against the closed form clamp(min(i+off+nxt, lk-1) - max(i+off-pre, 0) + 1, 0)
    for lq, lk, origin, pre, nxt in ((7, 12, 1, 3, 2), (9, 9, 0, 0, 0), (4, 10, 0, 2, -1), (6, 3, 1, 1, 5)):
        m = G.band_mask(lq, lk, origin, pre, nxt)
        off = lk - lq if origin else 0
        for i in range(lq):
            hi, lo = min(i + off + nxt, lk - 1), max(i + off - pre, 0)
            assert m[i].sum() == max(hi - lo + 1, 0)
            vis = [j for j in range(lk) if lo <= j <= hi]
            assert list(np.nonzero(m[i])[0]) == vis


def test_band_diagonal_returns_value_rows():
    q = RNG.standard_normal((1, 6, 2, 4)).astype(np.float32)
    k = RNG.standard_normal((1, 6, 1, 4)).astype(np.float32)
    v = RNG.standard_normal((1, 6, 1, 4)).astype(np.float32)
    out, lse = G.prefill_attention(q, k, v, None, None, 0, 0.5, band=(0, 0, 0))
    np.testing.assert_allclose(out[0, :, 0], v[0, :, 0], rtol=1e-6)
    np.testing.assert_allclose(lse[0, 0], (q[0, :, 0] * k[0, :, 0]).sum(-1) * 0.5, rtol=1e-5)
    # a band that leaves a query nothing gives zero output and lse -inf
    out, lse = G.prefill_attention(q, k, v, None, None, 0, 0.5, band=(0, 2147483647, -2))
    assert (out[0, :2] == 0).all() and np.isneginf(lse[0, :, :2]).all() and np.isfinite(lse[0, :, 2:]).all()


def test_paged_prefill_gather_and_decode_case():
    L, lq = [9, 14], [3, 5]
    bs, hkv, hq, d = 4, 2, 4, 8
    k, v, bt = _paged(L, hkv, d, bs, RNG)
    q = RNG.standard_normal((2, 5, hq, d)).astype(np.float32)
    out, lse = G.paged_prefill_attention(q, k, v, bt, lq, L, (1, 2147483647, 0), 0.3)
    for b in range(2):
        kk = k[bt[b]].reshape(-1, hkv, d)[None, :L[b]]
        vv = v[bt[b]].reshape(-1, hkv, d)[None, :L[b]]
        o2, l2 = G.prefill_attention(q[b:b + 1, :lq[b]], kk, vv, None, None, 1, 0.3)
        np.testing.assert_allclose(out[b, :lq[b]], o2[0], rtol=1e-6)
        np.testing.assert_allclose(lse[b, :, :lq[b]], l2[0], rtol=1e-6)
        assert (out[b, lq[b]:] == 0).all()
    # one query token with the bottom-right causal mask is the decode case
    o1, l1 = G.paged_prefill_attention(q[:, :1], k, v, bt, [1, 1], L, (1, 2147483647, 0), 0.3)
    od, ld = G.paged_decode_attention(q[:, 0], k, v, bt, L, 0.3)
    np.testing.assert_allclose(o1[:, 0], od, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(l1[:, :, 0], ld, rtol=1e-5)


def test_packed_tnd_attention_is_per_sequence_attention():
    # Each packed sequence attended alone (a batch of one, no length arguments) gives its rows; the
    # padding rows past the last end are zero with lse -inf; pack and unpack are inverses.
    lq, lk, hq, hkv, d = [3, 1, 5], [4, 7, 5], 4, 2, 8
    cq, ck = np.cumsum(lq), np.cumsum(lk)
    q = RNG.standard_normal((sum(lq) + 2, hq, d)).astype(np.float32)
    k = RNG.standard_normal((sum(lk), hkv, d)).astype(np.float32)
    v = RNG.standard_normal((sum(lk), hkv, d)).astype(np.float32)
    out, lse = G.packed_prefill_attention(q, k, v, cq, ck, 1, 0.4)
    for b in range(3):
        qs, ks = slice(cq[b] - lq[b], cq[b]), slice(ck[b] - lk[b], ck[b])
        o, l = G.prefill_attention(q[None, qs], k[None, ks], v[None, ks], None, None, 1, 0.4)
        np.testing.assert_allclose(out[qs], o[0], rtol=1e-6)
        np.testing.assert_allclose(lse[qs], l[0].T, rtol=1e-6)
    assert (out[sum(lq):] == 0).all() and np.isneginf(lse[sum(lq):]).all()
    np.testing.assert_array_equal(G.pack_tnd(G.unpack_tnd(k, ck, 7), lk), k)
    assert G.cum_to_lens([2, 2, 9]).tolist() == [2, 0, 7]


def test_mla_equals_gqa_on_dequantised_latent():
    L = [7, 20]
    bs, dn, dr, h = 4, 16, 4, 3
    nblk = 10
    ckv = RNG.integers(-127, 128, (nblk, bs, dn), dtype=np.int8)
    cs = RNG.uniform(1e-3, 1e-2, (nblk, bs)).astype(np.float32)
    kr = RNG.standard_normal((nblk, bs, dr)).astype(np.float32)
    bt = np.array([[3, 1, 0, 0, 0], [2, 5, 7, 9, 4]], np.int32)
    qn = RNG.standard_normal((2, h, dn)).astype(np.float32)
    qr = RNG.standard_normal((2, h, dr)).astype(np.float32)
    out, lse = G.mla_decode_attention(qn, qr, ckv, cs, kr, bt, L, 0.2)
    kfull = np.concatenate([ckv.astype(np.float32) * cs[..., None], kr], -1)[:, :, None, :]
    vfull = np.concatenate([ckv.astype(np.float32) * cs[..., None], np.zeros((nblk, bs, dr), np.float32)],
                           -1)[:, :, None, :]
    o2, l2 = G.paged_decode_attention(np.concatenate([qn, qr], -1), kfull, vfull, bt, L, 0.2)
    np.testing.assert_allclose(out, o2[..., :dn], rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(lse, l2, rtol=1e-5)


def test_dynamic_quant_v2_pinned():
    x = RNG.standard_normal((6, 40)).astype(np.float32) * 3
    x[2] = 0.0
    x[3] = np.abs(x[3]) + 0.5  # all positive: lo = 0
    # symmetric per token with q = 127 is the DynamicQuant rule
    y, s, off = G.dynamic_quant_v2(x)
    y0, s0 = G.dynamic_quant(x)
    np.testing.assert_array_equal(y, y0)
    np.testing.assert_array_equal(s, s0)
    assert off is None
    # a narrower symmetric range: max |y| = q, scale = amax / q
    y, s, _ = G.dynamic_quant_v2(x, dst_type_max=63.0)
    assert np.abs(y).max() == 63 and s[0] == pytest.approx(np.abs(x[0]).max() / 63, rel=1e-6)
    # per tensor = per token on the flattened input
    y, s, _ = G.dynamic_quant_v2(x, per_tensor=True)
    yf, sf = G.dynamic_quant(x.reshape(1, -1))
    np.testing.assert_array_equal(y, yf.reshape(x.shape))
    assert s.shape == (1,) and s[0] == sf[0]
    # asymmetric: the row extremes (range widened to 0) land on -128 / 127, reconstruction within half a step
    y, s, off = G.dynamic_quant_v2(x, symmetric=False)
    for r in (0, 1, 4, 5):
        assert y[r, np.argmin(x[r])] == -128 and y[r, np.argmax(x[r])] == 127
        rec = (y[r].astype(np.float64) - off[r]) * s[r]
        assert np.abs(rec - x[r]).max() <= s[r] * 0.5 * (1 + 1e-5)
    assert off[3] == pytest.approx(-128.0)  # lo = 0: offset -128
    assert s[2] == 0 and off[2] == 0 and (y[2] == 0).all()
    # asymmetric per tensor
    y, s, off = G.dynamic_quant_v2(x, symmetric=False, per_tensor=True)
    assert s.shape == (1,) and y.min() == -128 and y.max() == 127


def test_quant_matmul_int8_output_rule():
    x1 = RNG.integers(-127, 128, (9, 40), dtype=np.int8)
    x2 = RNG.integers(-127, 128, (40, 6), dtype=np.int8)
    acc = x1.astype(np.int64) @ x2.astype(np.int64)
    scale = np.full(6, 0.0625, np.float32)  # a power of two: acc * scale is exact
    off = np.array([0.0, 0.5, -0.5, 1.25, -3.0, 100.0], np.float32)
    got = G.quant_matmul(x1, x2, scale, None, None, "int8", offset=off)
    v = acc * 0.0625 + off.astype(np.float64)
    want = np.clip(np.round(v), -128, 127)  # numpy rounds half to even, like rint
    np.testing.assert_array_equal(got, want.astype(np.int8))


def test_explicit_mask_rule():
    q = RNG.standard_normal((2, 5, 2, 4)).astype(np.float32)
    k = RNG.standard_normal((2, 7, 1, 4)).astype(np.float32)
    v = RNG.standard_normal((2, 7, 1, 4)).astype(np.float32)
    big = 2147483647
    # the lower-triangle mask (1 above the diagonal) equals the top-left causal rule
    tri = np.triu(np.ones((5, 7), np.uint8), 1)[None]
    o1, l1 = G.prefill_attention(q, k, v, None, None, 0, 0.4, mask=tri)
    o2, l2 = G.prefill_attention(q, k, v, None, None, 2, 0.4)
    np.testing.assert_allclose(o1, o2, rtol=1e-6)
    np.testing.assert_allclose(l1, l2, rtol=1e-6)
    # a mask leaving one token per query returns that token's value row, per batch
    one = np.ones((2, 5, 7), np.uint8)
    pick = RNG.integers(0, 7, (2, 5))
    for b in range(2):
        one[b, np.arange(5), pick[b]] = 0
    o3, _ = G.prefill_attention(q, k, v, None, None, 0, 0.4, band=(0, big, big), mask=one)
    for b in range(2):
        np.testing.assert_allclose(o3[b, :, 0], v[b, pick[b], 0], rtol=1e-6)


# ----------------------------------------------------------------------------- int8 KV / int8 attention_out
def test_antiquant_kv_reductions():
    rng = np.random.default_rng(40)
    x = rng.integers(-128, 128, (2, 6, 3, 8)).astype(np.int8)
    # scale 1, offset 0: the integers themselves
    np.testing.assert_array_equal(G.antiquant_kv(x, np.ones(24)), x.astype(np.float32))
    # a per-channel scale that is one value everywhere equals a per-token scale of that value
    c = np.float32(0.0123)
    pc = G.antiquant_kv(x, np.full(24, c), np.full(24, 3.0), mode=0)
    pt = G.antiquant_kv(x, np.full((2, 9), c), np.full((2, 9), 3.0), mode=1)
    np.testing.assert_array_equal(pc, pt)
    # closed form of one element per mode: (x + offset) * scale
    sc = rng.random(24).astype(np.float32)
    of = rng.random(24).astype(np.float32)
    got = G.antiquant_kv(x, sc, of, mode=0)
    assert got[1, 4, 2, 5] == np.float32((np.float32(x[1, 4, 2, 5]) + of[2 * 8 + 5]) * sc[2 * 8 + 5])
    st = rng.random((2, 6)).astype(np.float32)
    so = rng.random((2, 6)).astype(np.float32)
    got = G.antiquant_kv(x, st, so, mode=1)
    assert got[0, 3, 1, 7] == np.float32((np.float32(x[0, 3, 1, 7]) + so[0, 3]) * st[0, 3])


def test_quant_attention_out_known_answers():
    o = np.array([0.5, 1.5, -2.5, 2.5, 200.0, -300.0, 0.49, -0.51], np.float32).reshape(1, 1, 1, 8)
    np.testing.assert_array_equal(G.quant_attention_out(o, [1.0]).reshape(-1), [0, 2, -2, 2, 127, -128, 0, -1])
    # per channel: channel h * D + d
    sc = np.arange(1, 9, dtype=np.float32)
    of = np.full(8, -0.25, np.float32)
    np.testing.assert_array_equal(G.quant_attention_out(np.ones((1, 1, 1, 8), np.float32), sc, of).reshape(-1),
                                  [1, 2, 3, 4, 5, 6, 7, 8])


def test_int8_kv_attention_reduces_to_float_attention_on_integer_values():
    """With scale 1 and offset 0 the int8 cache is the float attention over the integer values."""
    rng = np.random.default_rng(41)
    q = rng.standard_normal((1, 4, 2, 8)).astype(np.float32) * 0.1
    k = rng.integers(-128, 128, (1, 7, 1, 8)).astype(np.int8)
    v = rng.integers(-128, 128, (1, 7, 1, 8)).astype(np.int8)
    kd, vd = G.antiquant_kv(k, np.ones(8)), G.antiquant_kv(v, np.ones(8))
    out, lse = G.prefill_attention(q, kd, vd, None, None, 1, 0.3)
    want, wl = G.prefill_attention(q, k.astype(np.float32), v.astype(np.float32), None, None, 1, 0.3)
    np.testing.assert_array_equal(out, want)
    np.testing.assert_array_equal(lse, wl)


def test_mla_attention_with_one_query_token_is_mla_decode():
    rng = np.random.default_rng(42)
    b, h, dn, dr, bs = 3, 4, 16, 8, 4
    lens = [9, 1, 6]
    nblk = 8
    bt = np.stack([rng.permutation(nblk)[:3] for _ in range(b)]).astype(np.int32)
    qn = rng.standard_normal((b, h, dn)).astype(np.float32)
    qr = rng.standard_normal((b, h, dr)).astype(np.float32)
    ckv = rng.integers(-128, 128, (nblk, bs, dn)).astype(np.int8)
    cs = rng.random((nblk, bs)).astype(np.float32) * 0.01
    kr = rng.standard_normal((nblk, bs, dr)).astype(np.float32)
    want, wl = G.mla_decode_attention(qn, qr, ckv, cs, kr, bt, lens, 0.2)
    got, gl = G.mla_attention(qn[:, None], qr[:, None], ckv, cs, kr, bt, [1] * b, lens, (1, 2147483647, 0), 0.2)
    # (per-head against all-heads fp32 products: equal up to summation order)
    np.testing.assert_allclose(got[:, 0], want, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(gl[:, :, 0], wl, rtol=1e-6, atol=1e-6)
    # a later query token of a causal (bottom-right) sequence sees one more latent token than the one before
    got2, _ = G.mla_attention(np.repeat(qn[:, None], 2, 1), np.repeat(qr[:, None], 2, 1), ckv, cs, kr, bt, [2] * b,
                              lens, (1, 2147483647, 0), 0.2)
    np.testing.assert_allclose(got2[:, 1], want, rtol=1e-5, atol=1e-6)
    # the first of two tokens sees one latent token fewer: it equals decode over lens - 1
    want0, _ = G.mla_decode_attention(qn, qr, ckv, cs, kr, bt, [x - 1 for x in lens], 0.2)
    np.testing.assert_allclose(got2[:, 0], want0, rtol=1e-5, atol=1e-6)


def test_droppad_routing_against_dropless():
    rng = np.random.default_rng(43)
    t, k, e, h = 20, 3, 6, 4
    x = rng.standard_normal((t, h)).astype(np.float32)
    ei = rng.integers(0, e, (t, k)).astype(np.int32)
    dx, dri, dtok, _ = G.moe_init_routing_v2(x, ei, expert_start=0, expert_end=e, expert_tokens_num_type=1)
    cap = int(dtok.max())
    px, pri, ptok, _ = G.moe_init_routing_v2_droppad(x, ei, cap, expert_start=0, expert_end=e,
                                                     expert_tokens_num_type=1)
    np.testing.assert_array_equal(ptok, dtok)
    starts = np.concatenate([[0], np.cumsum(dtok)[:-1]])
    for ex_ in range(e):
        np.testing.assert_array_equal(px[ex_ * cap:ex_ * cap + dtok[ex_]], dx[starts[ex_]:starts[ex_] + dtok[ex_]])
        assert not px[ex_ * cap + dtok[ex_]:(ex_ + 1) * cap].any()
    # a slot's padded row = its expert's block + its dropless rank
    fe = ei.reshape(-1)
    np.testing.assert_array_equal(pri, fe * cap + (dri - starts[fe]))
    # capacity 1 keeps the first slot (in slot order) of every expert and drops the rest
    _, ri1, _, _ = G.moe_init_routing_v2_droppad(x, ei, 1, expert_start=0, expert_end=e)
    for ex_ in range(e):
        slots = np.nonzero(fe == ex_)[0]
        if len(slots):
            assert ri1[slots[0]] == ex_ and (ri1[slots[1:]] == -1).all()


def test_static_quant_rows_known_answers():
    x = np.array([[0.5, 1.5, -2.5, 300.0], [1.0, 2.0, 3.0, 4.0]], np.float32)
    np.testing.assert_array_equal(G.static_quant_rows(x, [1.0]), [[0, 2, -2, 127], [1, 2, 3, 4]])
    # per group, per column scale and offset: rint(x * s + o)
    sc = np.array([[1.0, 1.0, 1.0, 1.0], [2.0, 0.5, 1.0, -1.0]], np.float32)
    of = np.array([[0.0, 0.0, 0.0, 0.0], [0.25, 0.0, -0.5, 0.0]], np.float32)
    np.testing.assert_array_equal(G.static_quant_rows(x, sc, of, group_of_row=[1, 0]),
                                  [[1, 1, -3, -128], [1, 2, 3, 4]])


def test_dequant_swiglu_quant_static_known_answer():
    """quant_mode 0: clamp(rint(h * quant_scale + quant_offset)), scale 0; h from the dynamic path's
    composition (scale 1 / quant_scale 1 gives h itself)."""
    x = np.array([[10, -4, 3, 2]], np.int32)  # a = [10, -4], b = [3, 2]
    h = (G.silu(np.float32([10.0, -4.0])) * np.float32([3.0, 2.0])).astype(np.float32)
    y, s = G.dequant_swiglu_quant(x, activate_left=True, quant_mode=0, quant_scale=np.float32([2.0, 10.0]),
                                  quant_offset=np.float32([0.5, -1.0]))
    want = np.clip(np.rint(h * np.float32([2.0, 10.0]) + np.float32([0.5, -1.0])), -128, 127).astype(np.int8)
    np.testing.assert_array_equal(y, want.reshape(1, 2))
    assert s[0] == 0
    # saturation: h[0] ~ 30 times 10 is past 127, h[1] ~ -0.14 times 1000 is past -128
    y2, _ = G.dequant_swiglu_quant(x, activate_left=True, quant_mode=0, quant_scale=np.float32([10.0, 1000.0]))
    np.testing.assert_array_equal(y2, [[127, -128]])


def test_pse_shift_reductions():
    """pse = 0 is no pse; a pse constant along the kv axis changes nothing in the output (softmax shift)
    and adds itself to the lse; a -inf pse column masks that key out."""
    rng = np.random.default_rng(44)
    q = rng.standard_normal((2, 5, 4, 8)).astype(np.float32)
    k = rng.standard_normal((2, 7, 2, 8)).astype(np.float32)
    v = rng.standard_normal((2, 7, 2, 8)).astype(np.float32)
    base, bl = G.prefill_attention(q, k, v, None, None, 0, 0.3)
    z, zl = G.prefill_attention(q, k, v, None, None, 0, 0.3, pse=np.zeros((1, 4, 5, 7), np.float32))
    np.testing.assert_array_equal(z, base)
    np.testing.assert_array_equal(zl, bl)
    c = rng.standard_normal((2, 4, 5, 1)).astype(np.float32).repeat(7, axis=3)
    o, ol = G.prefill_attention(q, k, v, None, None, 0, 0.3, pse=c)
    np.testing.assert_allclose(o, base, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(ol, bl + c[:, :, :, 0], rtol=1e-5, atol=1e-5)
    m = np.zeros((1, 4, 5, 7), np.float32)
    m[..., 3] = -np.inf
    mask = np.zeros((1, 5, 7), np.uint8)
    mask[..., 3] = 1
    o2, _ = G.prefill_attention(q, k, v, None, None, 0, 0.3, pse=m)
    o3, _ = G.prefill_attention(q, k, v, None, None, 0, 0.3, mask=mask)
    np.testing.assert_array_equal(o2, o3)


def test_shared_prefix_reductions():
    """A shared prefix of length 0 changes nothing; when every sequence's keys start with the same
    rows, splitting those rows off into the shared prefix gives the same attention."""
    rng = np.random.default_rng(45)
    q = rng.standard_normal((2, 3, 4, 8)).astype(np.float32)
    k = rng.standard_normal((2, 9, 2, 8)).astype(np.float32)
    v = rng.standard_normal((2, 9, 2, 8)).astype(np.float32)
    lens = np.array([9, 6])
    kp, vp = rng.standard_normal((5, 2, 8)).astype(np.float32), rng.standard_normal((5, 2, 8)).astype(np.float32)
    k0, v0, l0 = G.with_shared_prefix(k, v, lens, kp, vp, 0)
    np.testing.assert_array_equal(k0[0], k[0])
    np.testing.assert_array_equal(v0[1, :6], v[1, :6])
    assert not k0[1, 6:].any()
    np.testing.assert_array_equal(l0, lens)
    k[:, :4], v[:, :4] = kp[:4], vp[:4]
    base, bl = G.prefill_attention(q, k, v, None, lens, 1, 0.3)
    kk, vv, ll = G.with_shared_prefix(k[:, 4:], v[:, 4:], lens - 4, kp, vp, 4)
    np.testing.assert_array_equal(ll, lens)
    o, ol = G.prefill_attention(q, kk, vv, None, ll, 1, 0.3)
    np.testing.assert_allclose(o, base, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(ol, bl, rtol=1e-6, atol=1e-6)


def test_swiglu_reductions():
    """b = 1 gives silu(a) = a * sigmoid(a) (scipy's expit); a = 0 gives 0; the split along another
    dimension equals the transposed last-dimension split."""
    from scipy.special import expit
    rng = np.random.default_rng(46)
    a = rng.standard_normal((5, 6)).astype(np.float32) * 4
    x = np.concatenate([a, np.ones_like(a)], axis=1)
    np.testing.assert_allclose(G.swiglu(x), a * expit(a), rtol=2e-6, atol=1e-7)
    x0 = np.concatenate([np.zeros_like(a), a], axis=1)
    assert not G.swiglu(x0).any()
    y = rng.standard_normal((8, 3)).astype(np.float32)
    np.testing.assert_array_equal(G.swiglu(y, dim=0), G.swiglu(y.T, dim=-1).T)
    assert G.swiglu(y.T, out_dtype="bf16").dtype == np.float32


def test_moe_compute_expert_tokens_brute_force():
    rng = np.random.default_rng(47)
    for n, e in ((0, 4), (50, 8), (300, 40)):
        se = np.sort(rng.integers(0, e + 3, n)).astype(np.int32)  # ids past the expert range too
        got = G.moe_compute_expert_tokens(se, e)
        want = np.array([(se <= k).sum() for k in range(e)], np.int32)
        np.testing.assert_array_equal(got, want)


def test_quant_query_attention_pins():
    # (1) one visible key: P = 1, P8 = rint(quant_scale1), O = P8 * v * dequant_scale2 exactly
    q = RNG.integers(-128, 128, (1, 3, 2, 16))
    k = RNG.integers(-128, 128, (1, 5, 1, 16))
    v = RNG.integers(-128, 128, (1, 5, 1, 16))
    big = 2147483647
    out, _ = G.quant_query_attention(q, k, v, 0.01, 100.0, 0.5, None, None, (0, 0, 0), 0.3)  # diagonal band
    for i in range(3):
        np.testing.assert_array_equal(out[0, i], np.broadcast_to(100 * v[0, i, 0] * 0.5, (2, 16)).astype(np.float32))
    # (2) against float attention: with quant_scale1 = 127 each P8 is within 0.5 of 127 * P, so
    #     O / (127 * dequant_scale2) differs from softmax attention by at most 0.5 * sum|v| / (127 * l)
    q = RNG.integers(-128, 128, (2, 6, 4, 32))
    k = RNG.integers(-128, 128, (2, 9, 2, 32))
    v = RNG.integers(-128, 128, (2, 9, 2, 32))
    d1, d2, sc = 1e-4, 0.02, 1 / math.sqrt(32)
    out, lse = G.quant_query_attention(q, k, v, d1, 127.0, d2, [6, 4], [9, 7], (1, big, 0), sc)
    ref, rl = G.prefill_attention((q * d1).astype(np.float32), k.astype(np.float32), v.astype(np.float32), [6, 4],
                                  [9, 7], 1, sc)
    bound = 0.5 * np.abs(v).sum(axis=1).max() / 127 + 1e-3
    assert np.abs(out / (127 * d2) - ref).max() <= bound
    assert np.abs(out / (127 * d2) - ref).max() > 0  # P really is quantised
    np.testing.assert_allclose(np.where(np.isfinite(lse), lse, 0), np.where(np.isfinite(rl), rl, 0), rtol=1e-5, atol=1e-5)
    # (3) identical value rows c: O = c * dequant_scale2 * sum(P8) / l
    vc = np.broadcast_to(RNG.integers(-128, 128, (1, 1, 1, 32)), (1, 9, 1, 32))
    out, _ = G.quant_query_attention(q[:1, :, :2], k[:1, :, :1], vc, d1, 90.0, d2, None, None, (0, big, big), sc)
    s = ((q[0, :, :2].astype(np.int64) @ k[0, :, 0].T.astype(np.int64)).astype(np.float32) * np.float32(d1)) * np.float32(sc)
    p = np.exp(s - s.max(-1, keepdims=True)).astype(np.float32)
    p8 = np.clip(np.rint(p * np.float32(90.0)), 0, 127)
    want = vc[0, 0, 0][None, None] * d2 * (p8.sum(-1) / p.sum(-1))[..., None]
    np.testing.assert_allclose(out[0], want, rtol=1e-5)


def test_learnable_sink_is_a_key_with_a_zero_value():
    # One query per batch row: a sink logit equals one more key, scored exactly that logit, whose value
    # row is zero; a sink at -inf is no sink.
    q = RNG.standard_normal((2, 1, 2, 8)).astype(np.float32)
    k = RNG.standard_normal((2, 5, 1, 8)).astype(np.float32)
    v = RNG.standard_normal((2, 5, 1, 8)).astype(np.float32)
    sink = np.array([0.7, -1.3], np.float32)
    out, lse = G.prefill_attention(q, k, v, None, None, 0, 0.5, sink=sink)
    for b in range(2):
        for h in range(2):
            qv = q[b, 0, h].astype(np.float64)
            kx = (qv * sink[h] / (0.5 * (qv @ qv)))[None]  # q . kx * 0.5 == sink[h]
            kk = np.concatenate([k[b, :, 0], kx.astype(np.float32)])
            vv = np.concatenate([v[b, :, 0], np.zeros((1, 8), np.float32)])
            o2, l2 = G.prefill_attention(q[b:b + 1, :, h:h + 1], kk[None, :, None], vv[None, :, None], None, None, 0,
                                         0.5)
            np.testing.assert_allclose(out[b, 0, h], o2[0, 0, 0], rtol=1e-5, atol=1e-6)
            np.testing.assert_allclose(lse[b, h, 0], l2[0, 0, 0], rtol=1e-5)
    o3, l3 = G.prefill_attention(q, k, v, None, None, 0, 0.5, sink=np.full(2, -np.inf, np.float32))
    o4, l4 = G.prefill_attention(q, k, v, None, None, 0, 0.5)
    np.testing.assert_array_equal(o3, o4)
    np.testing.assert_array_equal(l3, l4)


def test_dsq_swiglu_mode_1_pins():
    # (1) no clamping, glu_alpha 1, glu_bias 0: the odd-even mode is the halves mode on the de-interleaved
    #     columns (g * sigmoid(g) = silu(g))
    x = RNG.integers(-3000, 3000, (6, 16)).astype(np.int32)
    ws = RNG.uniform(1e-3, 2e-3, 16).astype(np.float32)
    act = RNG.uniform(0.5, 1.5, 6).astype(np.float32)
    perm = np.concatenate([np.arange(0, 16, 2), np.arange(1, 16, 2)])
    for left in (True, False):
        y1, s1 = G.dequant_swiglu_quant(x, ws, act, activate_left=left, swiglu_mode=1, clamp_limit=1e30,
                                        glu_alpha=1.0, glu_bias=0.0)
        y0, s0 = G.dequant_swiglu_quant(x[:, perm], ws[perm], act, activate_left=left)
        # (g * sigmoid(g) rounds sigmoid first, silu divides once: the two differ by an ulp at most)
        assert np.abs(y1.astype(int) - y0.astype(int)).max() <= 1
        np.testing.assert_allclose(s1, s0, rtol=2.5e-7, atol=0)
    # (2) the clamps, against float64 arithmetic: g = 10 -> 7, l = -9 -> -7 (limit 7, alpha 1.702, bias 1)
    xk = np.array([[10, -9, 2, 3]], np.int32)  # pairs (10, -9) and (2, 3); even activated (activate_left)
    y, s = G.dequant_swiglu_quant(xk, activate_left=True, swiglu_mode=1)
    h = [7 / (1 + math.exp(-1.702 * 7)) * (-7 + 1), 2 / (1 + math.exp(-1.702 * 2)) * (3 + 1)]
    assert abs(s[0] - max(abs(v) for v in h) / 127) <= 1e-6 * s[0]
    np.testing.assert_array_equal(y[0], np.rint(np.array(h) / s[0]).astype(np.int8))
