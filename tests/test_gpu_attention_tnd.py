"""npu_fused_infer_attention_score with packed (TND / NTD) queries: sequence b owns the query rows
[actual_seq_lengths[b-1], actual_seq_lengths[b]) (cumulative ends); dense keys/values are packed the
same way by actual_seq_lengths_kv, a paged cache takes per-sequence kv lengths. Output [T, N, D] (or
[N, T, D] for the NTD outputs) and lse [T, N, 1] follow the reference's TND shape rules
(python/torchair/ops/_npu_fused_infer_attention_score.py:171-180, 227-239, 300-327). Every case is
compared with the oracle's batched attention over the unpacked sequences."""
import math

import numpy as np
import pytest
import torch

import torchair_amd  # noqa: F401
from oracle import golden as G
from tests.helpers import assert_close, f32np

pytestmark = pytest.mark.gpu
DEV = "cuda"
FIA = torch.ops.npu.npu_fused_infer_attention_score


def _lse_np(x):
    x = np.asarray(x, np.float32)
    return np.where(np.isfinite(x), x, -1e30)


def _packed_inputs(g, lq, lk, hq, hkv, d, pad=3):
    tq, tk = sum(lq) + pad, sum(lk)
    q = torch.randn(tq, hq, d, generator=g).to(torch.bfloat16)
    k = torch.randn(tk, hkv, d, generator=g).to(torch.bfloat16)
    v = torch.randn(tk, hkv, d, generator=g).to(torch.bfloat16)
    return q, k, v


@pytest.mark.parametrize("layout", ["TND", "NTD", "TND_NTD", "NTD_TND"])
@pytest.mark.parametrize("cum_as_tensor", [False, True])
def test_dense_packed_prefill_causal(layout, cum_as_tensor):
    g = torch.Generator().manual_seed(170)
    lq, lk, hq, hkv, d = [33, 1, 70, 0], [33, 5, 90, 4], 8, 2, 128
    q, k, v = _packed_inputs(g, lq, lk, hq, hkv, d)
    cq, ck = np.cumsum(lq).tolist(), np.cumsum(lk).tolist()
    ql = layout[:3]
    tr = (lambda t: t) if ql == "TND" else (lambda t: t.transpose(0, 1).contiguous())
    lens = (lambda c: torch.tensor(c, device=DEV)) if cum_as_tensor else (lambda c: c)
    out, lse = FIA(tr(q).to(DEV), tr(k).to(DEV), tr(v).to(DEV), actual_seq_lengths=lens(cq),
                   actual_seq_lengths_kv=lens(ck), num_heads=hq, num_key_value_heads=hkv, input_layout=layout,
                   scale=1 / math.sqrt(d), sparse_mode=3, softmax_lse_flag=True)
    want, wl = G.packed_prefill_attention(f32np(q), f32np(k), f32np(v), cq, ck, 1, 1 / math.sqrt(d))
    tq = q.shape[0]
    ol = layout[-3:]
    assert out.shape == ((tq, hq, d) if ol == "TND" else (hq, tq, d)) and lse.shape == (tq, hq, 1)
    got = f32np(out) if ol == "TND" else f32np(out).transpose(1, 0, 2)
    assert_close(got, want)
    assert (got[sum(lq):] == 0).all()  # rows past the last end
    np.testing.assert_allclose(_lse_np(lse.cpu().numpy()[..., 0]), _lse_np(wl), rtol=1e-3, atol=1e-3)


def test_dense_packed_explicit_mask_and_int8_kv():
    """An explicit [B, Sq, Skv] mask indexed by position within each sequence, over int8 keys/values
    with per-channel antiquant scales."""
    g = torch.Generator().manual_seed(171)
    lq, lk, hq, hkv, d = [9, 17], [12, 17], 4, 1, 64
    tq, tk = sum(lq), sum(lk)
    q = torch.randn(tq, hq, d, generator=g).to(torch.bfloat16)
    k = torch.randint(-128, 128, (tk, hkv, d), generator=g, dtype=torch.int8)
    v = torch.randint(-128, 128, (tk, hkv, d), generator=g, dtype=torch.int8)
    ks, vs = torch.rand(hkv * d, generator=g) * 0.02 + 0.005, torch.rand(hkv * d, generator=g) * 0.02 + 0.005
    mask = torch.rand(2, 17, 17, generator=g) < 0.3
    mask[:, :, 0] = False  # every row sees kv 0
    cq, ck = np.cumsum(lq).tolist(), np.cumsum(lk).tolist()
    out, _ = FIA(q.to(DEV), k.to(DEV), v.to(DEV), atten_mask=mask.to(DEV), actual_seq_lengths=cq,
                 actual_seq_lengths_kv=ck, num_heads=hq, num_key_value_heads=hkv, input_layout="TND",
                 scale=1 / math.sqrt(d), sparse_mode=0, key_antiquant_scale=ks.to(DEV),
                 value_antiquant_scale=vs.to(DEV))
    kd = G.antiquant_kv(k.numpy()[None], ks.numpy(), None, 0)[0]
    vd = G.antiquant_kv(v.numpy()[None], vs.numpy(), None, 0)[0]
    want, _ = G.packed_prefill_attention(f32np(q), kd, vd, cq, ck, 0, 1 / math.sqrt(d), mask=mask.numpy())
    assert_close(f32np(out), want)


def _paged(lens, hkv, d, bs, g):
    b = len(lens)
    nb = [max((L + bs - 1) // bs, 1) for L in lens]
    total = sum(nb) + 2
    perm = torch.randperm(total, generator=g)
    bt = torch.zeros(b, max(nb), dtype=torch.int32)
    off = 0
    for i, n in enumerate(nb):
        bt[i, :n] = perm[off:off + n]
        off += n
    kc = torch.randn(total, bs, hkv, d, generator=g).to(torch.bfloat16)
    vc = torch.randn(total, bs, hkv, d, generator=g).to(torch.bfloat16)
    return kc, vc, bt


def test_paged_packed_chunked_prefill():
    """Packed query chunks over a paged cache (chunked prefill with mixed decode rows), bottom-right
    causal: the kv lengths are per sequence, the query ends cumulative."""
    g = torch.Generator().manual_seed(172)
    lq, lk, hq, hkv, d, bs = [1, 40, 3, 1], [100, 40, 260, 7], 16, 2, 128, 64
    kc, vc, bt = _paged(lk, hkv, d, bs, g)
    q = torch.randn(sum(lq), hq, d, generator=g).to(torch.bfloat16)
    cq = np.cumsum(lq).tolist()
    out, lse = FIA(q.to(DEV), kc.reshape(-1, bs, hkv * d).to(DEV), vc.reshape(-1, bs, hkv * d).to(DEV),
                   block_table=bt.to(DEV), actual_seq_lengths=torch.tensor(cq, device=DEV),
                   actual_seq_lengths_kv=torch.tensor(lk, device=DEV), num_heads=hq, num_key_value_heads=hkv,
                   input_layout="TND", block_size=bs, scale=1 / math.sqrt(d), sparse_mode=3, softmax_lse_flag=True)
    qb = G.unpack_tnd(f32np(q), cq, max(lq))
    o, l = G.paged_prefill_attention(qb, f32np(kc), f32np(vc), bt.numpy(), lq, lk, (1, 2147483647, 0),
                                     1 / math.sqrt(d))
    assert_close(f32np(out), G.pack_tnd(o, lq))
    np.testing.assert_allclose(_lse_np(lse.cpu().numpy()[..., 0]), _lse_np(G.pack_tnd(l.transpose(0, 2, 1), lq)),
                               rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("lens_kind", ["none", "list", "tensor"])
def test_paged_packed_one_token_each(lens_kind):
    """One query token per sequence: absent or host-list ends 1..B take the one-token kernel, device
    ends the general kernel; all agree with the oracle's decode."""
    g = torch.Generator().manual_seed(173)
    lk, hq, hkv, d, bs = [300, 1, 129, 64], 16, 4, 128, 64
    b = len(lk)
    kc, vc, bt = _paged(lk, hkv, d, bs, g)
    q = torch.randn(b, hq, d, generator=g).to(torch.bfloat16)
    kw = {}
    if lens_kind == "list":
        kw["actual_seq_lengths"] = list(range(1, b + 1))
    elif lens_kind == "tensor":
        kw["actual_seq_lengths"] = torch.arange(1, b + 1, device=DEV)
    out, lse = FIA(q.to(DEV), kc.reshape(-1, bs, hkv * d).to(DEV), vc.reshape(-1, bs, hkv * d).to(DEV),
                   block_table=bt.to(DEV), actual_seq_lengths_kv=lk, num_heads=hq, num_key_value_heads=hkv,
                   input_layout="TND", block_size=bs, scale=1 / math.sqrt(d), softmax_lse_flag=True, **kw)
    want, wl = G.paged_decode_attention(f32np(q), f32np(kc), f32np(vc), bt.numpy(), lk, 1 / math.sqrt(d))
    assert out.shape == (b, hq, d) and lse.shape == (b, hq, 1)
    assert_close(f32np(out), want)
    np.testing.assert_allclose(_lse_np(lse.cpu().numpy()[..., 0]), _lse_np(wl), rtol=1e-3, atol=1e-3)


def test_mla_int8_latent_packed_queries():
    """The int8 MLA latent with packed TND queries (MTP rows of different counts per sequence)."""
    g = torch.Generator().manual_seed(174)
    lq, lk, h, dn, dr, bs = [2, 1, 4], [300, 65, 7], 16, 512, 64, 64
    b = len(lk)
    nb = [(L + bs - 1) // bs for L in lk]
    total = sum(nb) + 2
    perm = torch.randperm(total, generator=g)
    bt = torch.zeros(b, max(nb), dtype=torch.int32)
    off = 0
    for i, n in enumerate(nb):
        bt[i, :n] = perm[off:off + n]
        off += n
    t = sum(lq)
    qn = torch.randn(t, h, dn, generator=g).to(torch.bfloat16)
    qr = torch.randn(t, h, dr, generator=g).to(torch.bfloat16)
    ckv = torch.randint(-128, 128, (total, bs, 1, dn), generator=g, dtype=torch.int8)
    cs = torch.rand(total, bs, generator=g) * 9e-3 + 1e-3
    kr = torch.randn(total, bs, 1, dr, generator=g).to(torch.bfloat16)
    scale = 1.0 / math.sqrt(192)
    cq = np.cumsum(lq).tolist()
    out, lse = FIA(qn.to(DEV), ckv.to(DEV), ckv.to(DEV), query_rope=qr.to(DEV), key_rope=kr.to(DEV),
                   key_antiquant_scale=cs.to(DEV), key_antiquant_mode=1, block_table=bt.to(DEV),
                   actual_seq_lengths=cq, actual_seq_lengths_kv=lk, num_heads=h, num_key_value_heads=1,
                   input_layout="TND", block_size=bs, scale=scale, softmax_lse_flag=True, sparse_mode=3)
    want, wl = G.mla_attention(G.unpack_tnd(f32np(qn), cq, max(lq)), G.unpack_tnd(f32np(qr), cq, max(lq)),
                               ckv[:, :, 0].numpy(), cs.numpy(), f32np(kr[:, :, 0]), bt.numpy(), lq, lk,
                               (1, 2147483647, 0), scale)
    assert out.shape == (t, h, dn) and lse.shape == (t, h, 1)
    assert_close(f32np(out), G.pack_tnd(want, lq))
    np.testing.assert_allclose(_lse_np(lse.cpu().numpy()[..., 0]), _lse_np(G.pack_tnd(wl.transpose(0, 2, 1), lq)),
                               rtol=1e-3, atol=1e-3)


def test_packed_layout_errors():
    q = torch.zeros(4, 2, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="actual_seq_lengths"):
        FIA(q, q, q, num_heads=2, input_layout="TND", actual_seq_lengths_kv=[4])
    with pytest.raises(RuntimeError, match="pse_shift"):
        FIA(q, q, q, num_heads=2, input_layout="TND", actual_seq_lengths=[4], actual_seq_lengths_kv=[4],
            pse_shift=torch.zeros(1, 2, 4, 4, dtype=torch.bfloat16, device=DEV))


@pytest.mark.parametrize("seed", range(6))
def test_dense_packed_random_shapes(seed):
    """Seeded random packed batches: 1-6 sequences (empty ones included), GQA ratios, head dims 64-256
    and the band / causal modes, against the oracle."""
    rng = np.random.default_rng(1000 + seed)
    g = torch.Generator().manual_seed(1000 + seed)
    b = int(rng.integers(1, 7))
    hkv = int(rng.choice([1, 2, 4]))
    hq = hkv * int(rng.choice([1, 2, 4]))
    d = int(rng.choice([64, 96, 128, 256]))
    lq = rng.integers(0, 40, b).tolist()
    lk = [int(x + rng.integers(0, 30)) for x in lq]
    mode = int(rng.choice([0, 2, 3, 4]))
    pre, nxt = int(rng.integers(1, 20)), int(rng.integers(0, 5))
    kw = dict(sparse_mode=mode)
    if mode in (0, 4):
        kw.update(pre_tokens=pre, next_tokens=nxt)
    band = {0: (0, pre, nxt), 2: (0, 2147483647, 0), 3: (1, 2147483647, 0), 4: (1, pre, nxt)}[mode]
    q, k, v = _packed_inputs(g, lq, lk, hq, hkv, d, pad=int(rng.integers(0, 3)))
    cq, ck = np.cumsum(lq).tolist(), np.cumsum(lk).tolist()
    out, lse = FIA(q.to(DEV), k.to(DEV), v.to(DEV), actual_seq_lengths=cq, actual_seq_lengths_kv=ck, num_heads=hq,
                   num_key_value_heads=hkv, input_layout="TND", scale=1 / math.sqrt(d), softmax_lse_flag=True, **kw)
    want, wl = G.packed_prefill_attention(f32np(q), f32np(k), f32np(v), cq, ck, 0, 1 / math.sqrt(d), band=band)
    assert_close(f32np(out), want)
    np.testing.assert_allclose(_lse_np(lse.cpu().numpy()[..., 0]), _lse_np(wl), rtol=1e-3, atol=1e-3)


def test_packed_int8_kv_and_int8_out():
    """Packed queries over int8 keys/values (per-channel scales) with an int8 attention_out."""
    g = torch.Generator().manual_seed(175)
    lq, lk, hq, hkv, d = [5, 0, 12], [9, 3, 12], 8, 2, 128
    tq, tk = sum(lq), sum(lk)
    q = torch.randn(tq, hq, d, generator=g).to(torch.bfloat16)
    k = torch.randint(-128, 128, (tk, hkv, d), generator=g, dtype=torch.int8)
    v = torch.randint(-128, 128, (tk, hkv, d), generator=g, dtype=torch.int8)
    ks, vs = torch.rand(hkv * d, generator=g) * 0.02 + 0.005, torch.rand(hkv * d, generator=g) * 0.02 + 0.005
    cq, ck = np.cumsum(lq).tolist(), np.cumsum(lk).tolist()
    out, _ = FIA(q.to(DEV), k.to(DEV), v.to(DEV), actual_seq_lengths=cq, actual_seq_lengths_kv=ck, num_heads=hq,
                 num_key_value_heads=hkv, input_layout="TND", scale=1 / math.sqrt(d), sparse_mode=3,
                 key_antiquant_scale=ks.to(DEV), value_antiquant_scale=vs.to(DEV),
                 quant_scale2=torch.tensor([40.0], device=DEV))
    kd = G.antiquant_kv(k.numpy()[None], ks.numpy(), None, 0)[0]
    vd = G.antiquant_kv(v.numpy()[None], vs.numpy(), None, 0)[0]
    want, _ = G.packed_prefill_attention(f32np(q), kd, vd, cq, ck, 1, 1 / math.sqrt(d))
    assert out.dtype == torch.int8 and out.shape == (tq, hq, d)
    exp8 = G.quant_attention_out(want[:, None], [40.0])[:, 0].astype(np.int32)
    assert np.abs(out.cpu().numpy().astype(np.int32) - exp8).max() <= 1


def test_packed_int8_query():
    """Packed int8 queries, keys and values with the three query-quant scales."""
    g = torch.Generator().manual_seed(176)
    lq, lk, hq, hkv, d = [3, 7], [20, 9], 4, 1, 64
    tq, tk = sum(lq), sum(lk)
    q = torch.randint(-128, 128, (tq, hq, d), generator=g, dtype=torch.int8)
    k = torch.randint(-128, 128, (tk, hkv, d), generator=g, dtype=torch.int8)
    v = torch.randint(-128, 128, (tk, hkv, d), generator=g, dtype=torch.int8)
    cq, ck = np.cumsum(lq).tolist(), np.cumsum(lk).tolist()
    d1, q1, d2 = 5e-4, 127.0, 1e-4
    out, _ = FIA(q.to(DEV), k.to(DEV), v.to(DEV), actual_seq_lengths=cq, actual_seq_lengths_kv=ck, num_heads=hq,
                 num_key_value_heads=hkv, input_layout="TND", scale=1 / math.sqrt(d), sparse_mode=3,
                 dequant_scale1=torch.tensor([d1], device=DEV), quant_scale1=torch.tensor([q1], device=DEV),
                 dequant_scale2=torch.tensor([d2], device=DEV))
    want, _ = G.quant_query_attention(G.unpack_tnd(q.numpy(), cq, max(lq)), G.unpack_tnd(k.numpy(), ck, max(lk)),
                                      G.unpack_tnd(v.numpy(), ck, max(lk)), d1, q1, d2, lq, lk, (1, 2147483647, 0),
                                      1 / math.sqrt(d))
    assert out.dtype == torch.float16
    # atol: one P8 rounding the other way between the device's and numpy's exp (see test_int8_query)
    assert_close(f32np(out), G.pack_tnd(want, lq), atol=2e-2)


def test_one_token_tnd_on_the_general_kernel_without_lengths():
    """A TND query of one token per sequence and no actual_seq_lengths, sent to the general kernel by an
    int8 attention_out: its cumulative ends are implied (1..B)."""
    g = torch.Generator().manual_seed(177)
    lk, hq, hkv, d, bs = [300, 1, 129, 64], 8, 2, 128, 64
    b = len(lk)
    kc, vc, bt = _paged(lk, hkv, d, bs, g)
    q = torch.randn(b, hq, d, generator=g).to(torch.bfloat16)
    out, _ = FIA(q.to(DEV), kc.reshape(-1, bs, hkv * d).to(DEV), vc.reshape(-1, bs, hkv * d).to(DEV),
                 block_table=bt.to(DEV), actual_seq_lengths_kv=lk, num_heads=hq, num_key_value_heads=hkv,
                 input_layout="TND", block_size=bs, scale=1 / math.sqrt(d), quant_scale2=torch.tensor([60.0], device=DEV))
    want, _ = G.paged_decode_attention(f32np(q), f32np(kc), f32np(vc), bt.numpy(), lk, 1 / math.sqrt(d))
    assert out.dtype == torch.int8 and out.shape == (b, hq, d)
    exp8 = G.quant_attention_out(want[:, None], [60.0])[:, 0].astype(np.int32)
    assert np.abs(out.cpu().numpy().astype(np.int32) - exp8).max() <= 1
