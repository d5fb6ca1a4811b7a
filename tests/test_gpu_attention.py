"""GPU parity: npu_fused_infer_attention_score (paged GQA decode, causal prefill, MLA decode)."""
import math

import numpy as np
import pytest
import torch

import torchair_amd  # noqa: F401
from oracle import golden as G
from tests.helpers import assert_close, f32np

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _paged_case(lens, hq, hkv, d, bs, seed, layout="BSH"):
    g = torch.Generator().manual_seed(seed)
    b = len(lens)
    nb = [(L + bs - 1) // bs for L in lens]
    total = sum(nb) + 3
    width = max(max(nb), 1)
    perm = torch.randperm(total, generator=g)
    bt = torch.zeros(b, width, dtype=torch.int32)
    off = 0
    for i, n in enumerate(nb):
        bt[i, :n] = perm[off:off + n]
        off += n
    k4 = torch.randn(total, bs, hkv, d, generator=g).to(torch.bfloat16)
    v4 = torch.randn(total, bs, hkv, d, generator=g).to(torch.bfloat16)
    q = torch.randn(b, hq, d, generator=g).to(torch.bfloat16)
    return q, k4, v4, bt, torch.tensor(lens, dtype=torch.int64)


def _decode(q, k4, v4, bt, lens, hq, hkv, d, bs, cache_layout="BSH", api="air", lse=True):
    b = q.shape[0]
    if cache_layout == "BSH":
        kc = k4.reshape(k4.shape[0], bs, hkv * d).to(DEV)
        vc = v4.reshape(v4.shape[0], bs, hkv * d).to(DEV)
    else:  # [blocks, Hkv, bs, D]
        kc = k4.permute(0, 2, 1, 3).contiguous().to(DEV)
        vc = v4.permute(0, 2, 1, 3).contiguous().to(DEV)
    qd = q.reshape(b, 1, hq * d).to(DEV)
    kw = dict(block_table=bt.to(DEV), num_heads=hq, num_key_value_heads=hkv, input_layout="BSH", block_size=bs,
              scale=1.0 / math.sqrt(d), softmax_lse_flag=lse)
    if api == "air":
        out, l = torch.ops.air.npu_fused_infer_attention_score(qd, kc, vc, actual_seq_lengths_kv=lens.to(DEV), **kw)
    else:
        out, l = torch.ops.npu.npu_fused_infer_attention_score(qd, kc, vc, actual_seq_lengths_kv=lens.tolist(), **kw)
    return out.reshape(b, hq, d), l


def _check_decode(lens, hq, hkv, d, bs, seed, **kw):
    q, k4, v4, bt, L = _paged_case(lens, hq, hkv, d, bs, seed)
    out, lse = _decode(q, k4, v4, bt, L, hq, hkv, d, bs, **kw)
    want, wl = G.paged_decode_attention(f32np(q), f32np(k4), f32np(v4), bt.numpy(), lens, 1.0 / math.sqrt(d))
    assert_close(f32np(out), want)
    wl_fin = np.where(np.isfinite(wl), wl, -1e30)
    got = lse.reshape(len(lens), hq).cpu().numpy()
    np.testing.assert_allclose(np.where(np.isfinite(got), got, -1e30), wl_fin, rtol=1e-3, atol=1e-3)


def test_paged_decode_cfg2():
    g = torch.Generator().manual_seed(100)
    lens = torch.randint(512, 4097, (64,), generator=g).tolist()
    _check_decode(lens, 32, 8, 128, 128, 101)


@pytest.mark.parametrize("hq,hkv,d", [(8, 8, 128), (16, 2, 64), (16, 1, 128), (4, 2, 256)])
def test_paged_decode_shapes(hq, hkv, d):
    _check_decode([1, 33, 300, 0, 257], hq, hkv, d, 64, 102)


def test_paged_decode_segments_longer_than_a_page_window():
    # 128 kv heads leave 8 step ranges, so a range covers ~74 pages of 32 tokens: the per-lane
    # block-table window (64 pages) has to move inside a segment
    _check_decode([12000, 7000, 0, 1], 128, 128, 64, 32, 104)


def test_paged_decode_bnsd_cache_and_list_lengths():
    _check_decode([77, 130, 512], 8, 2, 128, 32, 103, cache_layout="BNSD", api="npu", lse=True)


def _prefill_ref_torch(q, k, v, lq, lkv, causal, scale):
    """fp32 PyTorch reference on the GPU: q [B,S,Hq,D], k/v [B,S,Hkv,D]."""
    b, s, hq, d = q.shape
    hkv = k.shape[2]
    out = torch.zeros(b, s, hq, d, dtype=torch.float32, device=q.device)
    for i in range(b):
        a, c = int(lq[i]), int(lkv[i])
        qq = q[i, :a].float().permute(1, 0, 2)
        kk = k[i, :c].float().permute(1, 0, 2).repeat_interleave(hq // hkv, 0)
        vv = v[i, :c].float().permute(1, 0, 2).repeat_interleave(hq // hkv, 0)
        sc = (qq @ kk.transpose(1, 2)) * scale
        if causal:
            ii = torch.arange(a, device=q.device)[:, None]
            jj = torch.arange(c, device=q.device)[None, :]
            sc = sc.masked_fill(jj > ii + (c - a), float("-inf"))
        out[i, :a] = torch.softmax(sc, -1).matmul(vv).permute(1, 0, 2)
    return out


def _prefill(q, k, v, lq, lkv, hq, hkv, layout, sparse_mode, lse=False, **mask_kw):
    b, s = q.shape[0], q.shape[1]
    d = q.shape[3]
    if layout == "BSH":
        qa, ka, va = q.reshape(b, s, hq * d), k.reshape(b, k.shape[1], hkv * d), v.reshape(b, v.shape[1], hkv * d)
    elif layout == "BNSD":
        qa, ka, va = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    else:
        qa, ka, va = q, k, v
    out, l = torch.ops.air.npu_fused_infer_attention_score(
        qa, ka, va, actual_seq_lengths=lq.to(DEV), actual_seq_lengths_kv=lkv.to(DEV), num_heads=hq,
        num_key_value_heads=hkv, input_layout=layout, scale=1.0 / math.sqrt(d), sparse_mode=sparse_mode,
        softmax_lse_flag=lse, **mask_kw)
    if layout == "BSH":
        out = out.reshape(b, s, hq, d)
    elif layout == "BNSD":
        out = out.transpose(1, 2)
    return out, l


def test_prefill_cfg3_full_size():
    g = torch.Generator(device=DEV).manual_seed(110)
    b, s, hq, hkv, d = 4, 4096, 32, 8, 128
    q = torch.randn(b, s, hq, d, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(b, s, hkv, d, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(b, s, hkv, d, generator=g, device=DEV).to(torch.bfloat16)
    lens = torch.tensor([4096, 3072, 2048, 1024], dtype=torch.int64)
    out, _ = _prefill(q, k, v, lens, lens, hq, hkv, "BSH", 3)
    ref = _prefill_ref_torch(q, k, v, lens, lens, True, 1.0 / math.sqrt(d))
    for i in range(b):
        L = int(lens[i])
        torch.testing.assert_close(out[i, :L].float(), ref[i, :L], rtol=1e-2, atol=1e-2)
        assert (out[i, L:] == 0).all()


@pytest.mark.parametrize("layout", ["BSH", "BSND", "BNSD"])
@pytest.mark.parametrize("sparse_mode,causal", [(3, 1), (0, 0), (2, 2)])
def test_prefill_oracle(layout, sparse_mode, causal):
    gen = torch.Generator().manual_seed(111)
    b, s, hq, hkv, d = 3, 200, 8, 2, 64 if layout == "BNSD" else 128
    q = torch.randn(b, s, hq, d, generator=gen).to(torch.bfloat16)
    k = torch.randn(b, s, hkv, d, generator=gen).to(torch.bfloat16)
    v = torch.randn(b, s, hkv, d, generator=gen).to(torch.bfloat16)
    lq = torch.tensor([200, 150, 37])
    lkv = torch.tensor([200, 180, 37]) if causal != 2 else lq.clone()
    out, lse = _prefill(q.to(DEV), k.to(DEV), v.to(DEV), lq, lkv, hq, hkv, layout, sparse_mode, lse=True)
    want, wl = G.prefill_attention(f32np(q), f32np(k), f32np(v), lq.numpy(), lkv.numpy(), causal, 1.0 / math.sqrt(d))
    assert_close(f32np(out), want)
    got = lse.cpu().numpy().reshape(b, hq, s)
    np.testing.assert_allclose(np.where(np.isfinite(got), got, -1e30), np.where(np.isfinite(wl), wl, -1e30),
                               rtol=1e-3, atol=1e-3)


def _mla_case(lens, h, bs, seed):
    g = torch.Generator().manual_seed(seed)
    b = len(lens)
    nb = [(L + bs - 1) // bs for L in lens]
    total = sum(nb) + 2
    perm = torch.randperm(total, generator=g)
    bt = torch.zeros(b, max(nb), dtype=torch.int32)
    off = 0
    for i, n in enumerate(nb):
        bt[i, :n] = perm[off:off + n]
        off += n
    qn = torch.randn(b, 1, h, 512, generator=g).to(torch.bfloat16)
    qr = torch.randn(b, 1, h, 64, generator=g).to(torch.bfloat16)
    ckv = torch.randint(-127, 128, (total, bs, 1, 512), generator=g, dtype=torch.int8)
    cs = torch.rand(total, bs, generator=g) * 9e-3 + 1e-3
    kr = torch.randn(total, bs, 1, 64, generator=g).to(torch.bfloat16)
    return qn, qr, ckv, cs, kr, bt


def _check_mla(lens, h, bs, seed):
    qn, qr, ckv, cs, kr, bt = _mla_case(lens, h, bs, seed)
    scale = 1.0 / math.sqrt(192)
    out, lse = torch.ops.air.npu_fused_infer_attention_score(
        qn.to(DEV), ckv.to(DEV), ckv.to(DEV), query_rope=qr.to(DEV), key_rope=kr.to(DEV),
        key_antiquant_scale=cs.to(DEV), key_antiquant_mode=1, block_table=bt.to(DEV),
        actual_seq_lengths_kv=torch.tensor(lens, device=DEV), num_heads=h, num_key_value_heads=1,
        input_layout="BSND", block_size=bs, scale=scale, softmax_lse_flag=True)
    assert out.shape == (len(lens), 1, h, 512)
    want, wl = G.mla_decode_attention(f32np(qn[:, 0]), f32np(qr[:, 0]), ckv[:, :, 0].numpy(), cs.numpy(),
                                      f32np(kr[:, :, 0]), bt.numpy(), lens, scale)
    assert_close(f32np(out[:, 0]), want)
    got = lse.reshape(len(lens), h).cpu().numpy()
    np.testing.assert_allclose(np.where(np.isfinite(got), got, -1e30), np.where(np.isfinite(wl), wl, -1e30),
                               rtol=1e-3, atol=1e-3)


def test_mla_small():
    _check_mla([1, 40, 1100, 0, 2049], 128, 64, 120)


def test_mla_small_pages_long_split():
    # block_size 32: a full split spans 64 pages (one page id per lane)
    _check_mla([4100, 2048, 31], 16, 32, 123)


def test_mla_cfg5():
    g = torch.Generator().manual_seed(121)
    lens = torch.randint(2048, 8193, (128,), generator=g).tolist()
    _check_mla(lens, 128, 128, 122)


def test_mla_rising_logits_take_the_rescaling_pass():
    # Every third page of sequence 0 has rope keys whose logits exceed the others by ~200 (log2
    # units): past the fast pass's headroom, so P' would overflow bf16. The fast pass flags the
    # segments where such a page follows a low one and the rescaling pass redoes them; the other
    # segments and sequences stay on the fast pass.
    lens, h, bs = [30000, 500, 2100], 128, 64
    qn, qr, ckv, cs, kr, bt = _mla_case(lens, h, bs, 124)
    qr = torch.ones_like(qr)
    for j in range(2, (lens[0] + bs - 1) // bs, 3):
        kr[bt[0, j]] = 32.0
    scale = 1.0 / math.sqrt(192)
    out, lse = torch.ops.air.npu_fused_infer_attention_score(
        qn.to(DEV), ckv.to(DEV), ckv.to(DEV), query_rope=qr.to(DEV), key_rope=kr.to(DEV),
        key_antiquant_scale=cs.to(DEV), key_antiquant_mode=1, block_table=bt.to(DEV),
        actual_seq_lengths_kv=torch.tensor(lens, device=DEV), num_heads=h, num_key_value_heads=1,
        input_layout="BSND", block_size=bs, scale=scale, softmax_lse_flag=True)
    want, wl = G.mla_decode_attention(f32np(qn[:, 0]), f32np(qr[:, 0]), ckv[:, :, 0].numpy(), cs.numpy(),
                                      f32np(kr[:, :, 0]), bt.numpy(), lens, scale)
    assert np.isfinite(f32np(out)).all()
    assert_close(f32np(out[:, 0]), want)
    got = lse.reshape(len(lens), h).cpu().numpy()
    np.testing.assert_allclose(got, wl, rtol=1e-3, atol=1e-3)


def test_mla_segments_longer_than_a_page_window():
    # block_size 32 and ~16.9K steps over 256 workgroups: ~66 steps (= pages) per workgroup range, so
    # segments cross the 64-page window of page ids the kernel holds and reload it
    lens, h, bs = [140000, 140000, 140000, 120000], 16, 32
    _check_mla(lens, h, bs, 125)


@pytest.mark.parametrize("d", [64, 128])
def test_prefill_rising_logits_take_the_rescaling_loop(d):
    # Keys grow along the sequence, so a query's logits rise by far more than the fast loop's 2^64
    # headroom (log2 units) above the max of the first tile it sees: those waves switch to the
    # rescaling loop mid-sequence. Batch 1 keeps random keys (fast loop only).
    gen = torch.Generator().manual_seed(112)
    b, s, hq, hkv = 2, 333, 4, 2
    q = torch.randn(b, s, hq, d, generator=gen).to(torch.bfloat16)
    k = torch.randn(b, s, hkv, d, generator=gen).to(torch.bfloat16)
    v = torch.randn(b, s, hkv, d, generator=gen).to(torch.bfloat16)
    q[0] = 1.0
    k[0] = (torch.arange(s, dtype=torch.float32) * (12.0 / s)).view(s, 1, 1).expand(s, hkv, d).to(torch.bfloat16)
    lens = torch.tensor([s, 250])
    for sparse_mode, causal in ((3, 1), (0, 0)):
        out, lse = _prefill(q.to(DEV), k.to(DEV), v.to(DEV), lens, lens, hq, hkv, "BSND", sparse_mode, lse=True)
        want, wl = G.prefill_attention(f32np(q), f32np(k), f32np(v), lens.numpy(), lens.numpy(), causal,
                                       1.0 / math.sqrt(d))
        assert np.isfinite(f32np(out)).all()
        assert_close(f32np(out), want)
        got = lse.cpu().numpy().reshape(b, hq, s)
        fin = np.isfinite(wl)
        np.testing.assert_array_equal(np.isfinite(got), fin)
        np.testing.assert_allclose(got[fin], wl[fin], rtol=1e-3, atol=1e-3)


def _assert_lse(got, wl):
    """lse: -inf exactly where the oracle's is, elsewhere the fp32-output bar (rtol = atol = 1e-2). The
    kernel's row sums add the bf16-rounded P that also feeds P V, so a row of a few visible tokens can
    differ by ~2^-9 relative per term."""
    fin = np.isfinite(wl)
    np.testing.assert_array_equal(np.isfinite(got), fin)
    np.testing.assert_allclose(got[fin], wl[fin], rtol=1e-2, atol=1e-2)


# Band masks (sparse_mode 0: pre/next tokens from the top-left; 4: from the bottom-right), including a
# band that leaves the first queries nothing (next_tokens < 0) and one narrower than a 32-token step.
@pytest.mark.parametrize("sparse_mode,pre,nxt", [(0, 50, 7), (0, 2147483647, -10), (0, 5, 0), (4, 20, 0),
                                                 (4, 100, 30), (4, 0, 0)])
def test_prefill_band_masks(sparse_mode, pre, nxt):
    gen = torch.Generator().manual_seed(113)
    b, s, hq, hkv, d = 2, 230, 8, 2, 128
    q = torch.randn(b, s, hq, d, generator=gen).to(torch.bfloat16)
    k = torch.randn(b, s, hkv, d, generator=gen).to(torch.bfloat16)
    v = torch.randn(b, s, hkv, d, generator=gen).to(torch.bfloat16)
    lq, lkv = torch.tensor([230, 101]), torch.tensor([230, 199])
    out, lse = _prefill(q.to(DEV), k.to(DEV), v.to(DEV), lq, lkv, hq, hkv, "BSND", sparse_mode, lse=True,
                        pre_tokens=pre, next_tokens=nxt)
    band = (1 if sparse_mode == 4 else 0, pre, nxt)
    want, wl = G.prefill_attention(f32np(q), f32np(k), f32np(v), lq.numpy(), lkv.numpy(), 0, 1.0 / math.sqrt(d),
                                   band=band)
    assert_close(f32np(out), want)
    _assert_lse(lse.cpu().numpy().reshape(b, hq, s), wl)


def _paged_seq_case(lq, lkv, hq, hkv, d, bs, seed):
    g = torch.Generator().manual_seed(seed)
    b = len(lkv)
    nb = [(L + bs - 1) // bs for L in lkv]
    total = sum(nb) + 3
    perm = torch.randperm(total, generator=g)
    bt = torch.zeros(b, max(nb), dtype=torch.int32)
    off = 0
    for i, n in enumerate(nb):
        bt[i, :n] = perm[off:off + n]
        off += n
    k4 = torch.randn(total, bs, hkv, d, generator=g).to(torch.bfloat16)
    v4 = torch.randn(total, bs, hkv, d, generator=g).to(torch.bfloat16)
    q = torch.randn(b, max(lq), hq, d, generator=g).to(torch.bfloat16)
    return q, k4, v4, bt


def _paged_seq(q, k4, v4, bt, lq, lkv, hq, hkv, bs, q_layout, cache_layout, **mask_kw):
    b, s, _, d = q.shape
    if cache_layout == "BSH":
        kc = k4.reshape(k4.shape[0], bs, hkv * d).to(DEV)
        vc = v4.reshape(v4.shape[0], bs, hkv * d).to(DEV)
    else:  # [blocks, Hkv, bs, D]
        kc = k4.permute(0, 2, 1, 3).contiguous().to(DEV)
        vc = v4.permute(0, 2, 1, 3).contiguous().to(DEV)
    if q_layout == "BSH":
        qa = q.reshape(b, s, hq * d)
    elif q_layout == "BNSD":
        qa = q.transpose(1, 2)
    else:
        qa = q
    out, l = torch.ops.air.npu_fused_infer_attention_score(
        qa.to(DEV), kc, vc, block_table=bt.to(DEV), actual_seq_lengths=torch.tensor(lq, device=DEV),
        actual_seq_lengths_kv=torch.tensor(lkv, device=DEV), num_heads=hq, num_key_value_heads=hkv,
        input_layout=q_layout, block_size=bs, scale=1.0 / math.sqrt(d), softmax_lse_flag=True, **mask_kw)
    if q_layout == "BSH":
        out = out.reshape(b, s, hq, d)
    elif q_layout == "BNSD":
        out = out.transpose(1, 2)
    return out, l


# Chunked prefill over a paged cache: each sequence's new query tokens are the last len_q of its len_kv
# tokens (bottom-right causal, sparse_mode 3); block sizes 32 / 64 / 128 / 96 (a 64-token tile across
# two blocks), both cache layouts, the three query layouts.
@pytest.mark.parametrize("bs,cache_layout,q_layout", [(128, "BSH", "BSH"), (64, "BNSD", "BSND"), (32, "BSH", "BNSD"),
                                                      (96, "BNSD", "BSH")])
def test_paged_chunked_prefill(bs, cache_layout, q_layout):
    lq, lkv = [37, 64, 1, 100], [300, 64, 77, 229]
    hq, hkv, d = 8, 2, 128
    q, k4, v4, bt = _paged_seq_case(lq, lkv, hq, hkv, d, bs, 114)
    out, lse = _paged_seq(q, k4, v4, bt, lq, lkv, hq, hkv, bs, q_layout, cache_layout, sparse_mode=3)
    want, wl = G.paged_prefill_attention(f32np(q), f32np(k4), f32np(v4), bt.numpy(), lq, lkv, (1, 2147483647, 0),
                                         1.0 / math.sqrt(d))
    assert_close(f32np(out), want)
    _assert_lse(lse.cpu().numpy().reshape(len(lq), hq, max(lq)), wl)


# Multi-token decode (speculative / MTP: 2-4 new tokens per sequence) and a sliding window over the
# paged cache (sparse_mode 4, including one query token, which then takes the query-sequence kernel).
@pytest.mark.parametrize("lq,mask_kw,band", [
    ([3, 2, 4], dict(sparse_mode=3), (1, 2147483647, 0)),
    ([4, 4, 4], dict(sparse_mode=4, pre_tokens=40, next_tokens=0), (1, 40, 0)),
    ([1, 1, 1], dict(sparse_mode=4, pre_tokens=70, next_tokens=0), (1, 70, 0)),
])
def test_paged_multi_token_decode_and_window(lq, mask_kw, band):
    lkv = [517, 130, 64]
    hq, hkv, d, bs = 32, 8, 128, 128
    q, k4, v4, bt = _paged_seq_case(lq, lkv, hq, hkv, d, bs, 115)
    out, lse = _paged_seq(q, k4, v4, bt, lq, lkv, hq, hkv, bs, "BSH", "BSH", **mask_kw)
    want, wl = G.paged_prefill_attention(f32np(q), f32np(k4), f32np(v4), bt.numpy(), lq, lkv, band,
                                         1.0 / math.sqrt(d))
    assert_close(f32np(out), want)
    _assert_lse(lse.cpu().numpy().reshape(len(lq), hq, max(lq)), wl)


# fp16 query / key / value: the MFMAs take fp16 on both operands (P rounded to fp16), the fast
# prefill pass keeps P within 2^8 of its reference max.
def test_paged_decode_fp16():
    lens, hq, hkv, d, bs = [700, 33, 1, 129], 32, 8, 128, 128
    q, k4, v4, bt, L = _paged_case(lens, hq, hkv, d, bs, 116)
    q, k4, v4 = q.half(), k4.half(), v4.half()
    out, lse = _decode(q, k4, v4, bt, L, hq, hkv, d, bs)
    assert out.dtype == torch.float16
    want, wl = G.paged_decode_attention(f32np(q), f32np(k4), f32np(v4), bt.numpy(), lens, 1.0 / math.sqrt(d))
    assert_close(f32np(out), want)
    _assert_lse(lse.reshape(len(lens), hq).cpu().numpy(), wl)


@pytest.mark.parametrize("sparse_mode,band", [(3, (1, 2147483647, 0)), (4, (1, 40, 3))])
def test_prefill_fp16(sparse_mode, band):
    gen = torch.Generator().manual_seed(117)
    b, s, hq, hkv, d = 2, 190, 8, 2, 128
    q = torch.randn(b, s, hq, d, generator=gen).half()
    k = torch.randn(b, s, hkv, d, generator=gen).half()
    v = torch.randn(b, s, hkv, d, generator=gen).half()
    lq, lkv = torch.tensor([190, 77]), torch.tensor([190, 120])
    kw = dict(pre_tokens=band[1], next_tokens=band[2]) if sparse_mode == 4 else {}
    out, lse = _prefill(q.to(DEV), k.to(DEV), v.to(DEV), lq, lkv, hq, hkv, "BSND", sparse_mode, lse=True, **kw)
    assert out.dtype == torch.float16
    want, wl = G.prefill_attention(f32np(q), f32np(k), f32np(v), lq.numpy(), lkv.numpy(), 0, 1.0 / math.sqrt(d),
                                   band=band)
    assert_close(f32np(out), want)
    _assert_lse(lse.cpu().numpy().reshape(b, hq, s), wl)


def test_prefill_fp16_rising_logits_take_the_rescaling_pass():
    # logits rising far beyond the fp16 fast pass's 2^8 headroom: its items are redone by the rescaling pass
    gen = torch.Generator().manual_seed(118)
    b, s, hq, hkv, d = 1, 300, 4, 2, 64
    q = torch.ones(b, s, hq, d).half()
    k = (torch.arange(s, dtype=torch.float32) * (6.0 / s)).view(1, s, 1, 1).expand(b, s, hkv, d).half()
    v = torch.randn(b, s, hkv, d, generator=gen).half()
    lens = torch.tensor([s])
    out, lse = _prefill(q.to(DEV), k.to(DEV), v.to(DEV), lens, lens, hq, hkv, "BSND", 3, lse=True)
    want, wl = G.prefill_attention(f32np(q), f32np(k), f32np(v), lens.numpy(), lens.numpy(), 1, 1.0 / math.sqrt(d))
    assert np.isfinite(f32np(out)).all()
    assert_close(f32np(out), want)
    _assert_lse(lse.cpu().numpy().reshape(b, hq, s), wl)


# Explicit atten_mask (sparse_mode 1, and 0 with a band), head dims the tiled kernels do not take, and an
# MLA latent in bf16: the general kernel.
@pytest.mark.parametrize("sparse_mode,mask_shape,band", [(1, "B1SS", None), (0, "SS", (0, 60, 5)), (0, "BSS", None)])
def test_prefill_explicit_mask(sparse_mode, mask_shape, band):
    gen = torch.Generator().manual_seed(119)
    b, s, hq, hkv, d = 2, 150, 8, 2, 128
    q = torch.randn(b, s, hq, d, generator=gen).to(torch.bfloat16)
    k = torch.randn(b, s, hkv, d, generator=gen).to(torch.bfloat16)
    v = torch.randn(b, s, hkv, d, generator=gen).to(torch.bfloat16)
    full = torch.rand(b, s, s, generator=gen) < 0.3
    full[:, 5, :] = True  # a query that sees nothing
    mask = {"B1SS": full[:, None], "SS": full[0], "BSS": full}[mask_shape]
    lq, lkv = torch.tensor([150, 90]), torch.tensor([150, 120])
    kw = dict(atten_mask=mask.to(DEV))
    if band is not None:
        kw.update(pre_tokens=band[1], next_tokens=band[2])
    out, lse = _prefill(q.to(DEV), k.to(DEV), v.to(DEV), lq, lkv, hq, hkv, "BSND", sparse_mode, lse=True, **kw)
    m3 = mask.numpy().reshape(-1, s, s)
    want, wl = G.prefill_attention(f32np(q), f32np(k), f32np(v), lq.numpy(), lkv.numpy(), 0, 1.0 / math.sqrt(d),
                                   band=band, mask=m3.astype(np.uint8))
    assert_close(f32np(out), want)
    _assert_lse(lse.cpu().numpy().reshape(b, hq, s), wl)


@pytest.mark.parametrize("d", [96, 192])
def test_prefill_other_head_dims(d):
    gen = torch.Generator().manual_seed(120)
    b, s, hq, hkv = 2, 70, 4, 2
    q = torch.randn(b, s, hq, d, generator=gen).half()
    k = torch.randn(b, s, hkv, d, generator=gen).half()
    v = torch.randn(b, s, hkv, d, generator=gen).half()
    lens = torch.tensor([70, 33])
    out, lse = _prefill(q.to(DEV), k.to(DEV), v.to(DEV), lens, lens, hq, hkv, "BSND", 3, lse=True)
    want, wl = G.prefill_attention(f32np(q), f32np(k), f32np(v), lens.numpy(), lens.numpy(), 1, 1.0 / math.sqrt(d))
    assert_close(f32np(out), want)
    _assert_lse(lse.cpu().numpy().reshape(b, hq, s), wl)


def test_paged_explicit_mask():
    lq, lkv = [3, 1], [200, 77]
    hq, hkv, d, bs = 8, 2, 128, 64
    q, k4, v4, bt = _paged_seq_case(lq, lkv, hq, hkv, d, bs, 121)
    gen = torch.Generator().manual_seed(122)
    mask = torch.rand(2, 1, 3, 200, generator=gen) < 0.5
    out, lse = _paged_seq(q, k4, v4, bt, lq, lkv, hq, hkv, bs, "BSH", "BSH", sparse_mode=1, atten_mask=mask.to(DEV))
    want, wl = G.paged_prefill_attention(f32np(q), f32np(k4), f32np(v4), bt.numpy(), lq, lkv,
                                         (0, 2147483647, 2147483647), 1.0 / math.sqrt(d),
                                         mask=mask[:, 0].numpy().astype(np.uint8))
    assert_close(f32np(out), want)
    _assert_lse(lse.cpu().numpy().reshape(2, hq, 3), wl)


@pytest.mark.parametrize("lq", [1, 3])
def test_paged_small_blocks(lq):
    """Block sizes that are not a multiple of 32 tokens take the general kernel."""
    lqs, lkv = [lq, 1], [100, 37]
    hq, hkv, d, bs = 8, 2, 128, 16
    q, k4, v4, bt = _paged_seq_case(lqs, lkv, hq, hkv, d, bs, 125)
    out, lse = _paged_seq(q, k4, v4, bt, lqs, lkv, hq, hkv, bs, "BSH", "BSH", sparse_mode=3)
    want, wl = G.paged_prefill_attention(f32np(q), f32np(k4), f32np(v4), bt.numpy(), lqs, lkv,
                                         (1, 2147483647, 0), 1.0 / math.sqrt(d))
    assert_close(f32np(out), want)
    _assert_lse(lse.cpu().numpy().reshape(2, hq, lq), wl)


def test_mla_bf16_latent():
    lens, h, bs = [300, 65, 1], 16, 64
    qn, qr, ckv, cs, kr, bt = _mla_case(lens, h, bs, 123)
    lat = (torch.randn(ckv.shape, generator=torch.Generator().manual_seed(124)) * 0.5).to(torch.bfloat16)
    scale = 1.0 / math.sqrt(192)
    out, lse = torch.ops.air.npu_fused_infer_attention_score(
        qn.to(DEV), lat.to(DEV), lat.to(DEV), query_rope=qr.to(DEV), key_rope=kr.to(DEV), block_table=bt.to(DEV),
        actual_seq_lengths_kv=torch.tensor(lens, device=DEV), num_heads=h, num_key_value_heads=1,
        input_layout="BSND", block_size=bs, scale=scale, softmax_lse_flag=True)
    assert out.shape == (len(lens), 1, h, 512) and out.dtype == torch.bfloat16
    ones = np.ones(cs.shape, np.float32)
    want, wl = G.mla_decode_attention(f32np(qn[:, 0]), f32np(qr[:, 0]), f32np(lat[:, :, 0]), ones, f32np(kr[:, :, 0]),
                                      bt.numpy(), lens, scale)
    assert_close(f32np(out[:, 0]), want)
    _assert_lse(lse.reshape(len(lens), h).cpu().numpy(), wl)
