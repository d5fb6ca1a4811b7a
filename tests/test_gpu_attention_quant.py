"""GPU parity: npu_fused_infer_attention_score with int8 key / value caches (antiquant scales and
offsets, per channel and per token, the separate key_/value_ and the combined antiquant_* forms)
and with int8 attention_out (quant_scale2 / quant_offset2), against the oracle: attention over the
dequantised caches (oracle.golden.antiquant_kv), then quant_attention_out for the int8 output.
Bars: bf16 outputs rtol = atol = 1e-2; int8 outputs within 1 LSB on at most 0.1% of elements."""
import math

import numpy as np
import pytest
import torch

import torchair_amd  # noqa: F401
from oracle import golden as G
from tests.helpers import assert_close, assert_int8_close, f32np

pytestmark = pytest.mark.gpu
DEV = "cuda"
FIA = torch.ops.npu.npu_fused_infer_attention_score


def _i8(shape, g):
    return torch.randint(-128, 128, shape, generator=g, dtype=torch.int8)


def _lse(lse, b, hq, s):
    got = lse.cpu().numpy().reshape(b, hq, s)
    return np.where(np.isfinite(got), got, -1e30)


@pytest.mark.parametrize("with_offset", [False, True])
def test_dense_prefill_int8_kv_per_channel(with_offset):
    g = torch.Generator().manual_seed(150)
    b, s, hq, hkv, d = 2, 96, 8, 2, 128
    q = torch.randn(b, s, hq, d, generator=g).to(torch.bfloat16)
    k, v = _i8((b, s, hkv, d), g), _i8((b, s, hkv, d), g)
    ks = torch.rand(hkv * d, generator=g) * 0.02 + 0.005
    vs = torch.rand(hkv * d, generator=g) * 0.02 + 0.005
    ko = (torch.rand(hkv * d, generator=g) * 4 - 2) if with_offset else None
    vo = (torch.rand(hkv * d, generator=g) * 4 - 2) if with_offset else None
    lens = [96, 50]
    kw = dict(key_antiquant_scale=ks.to(DEV), value_antiquant_scale=vs.to(DEV))
    if with_offset:
        kw.update(key_antiquant_offset=ko.to(DEV), value_antiquant_offset=vo.to(DEV))
    out, lse = FIA(q.reshape(b, s, hq * d).to(DEV), k.reshape(b, s, hkv * d).to(DEV), v.reshape(b, s, hkv * d).to(DEV),
                   actual_seq_lengths=lens, actual_seq_lengths_kv=lens, num_heads=hq, num_key_value_heads=hkv,
                   input_layout="BSH", scale=1 / math.sqrt(d), sparse_mode=3, softmax_lse_flag=True, **kw)
    kd = G.antiquant_kv(k.numpy(), ks.numpy(), None if ko is None else ko.numpy(), 0)
    vd = G.antiquant_kv(v.numpy(), vs.numpy(), None if vo is None else vo.numpy(), 0)
    want, wl = G.prefill_attention(f32np(q), kd, vd, np.array(lens), np.array(lens), 1, 1 / math.sqrt(d))
    assert out.dtype == torch.bfloat16
    assert_close(f32np(out.reshape(b, s, hq, d)), want)
    np.testing.assert_allclose(_lse(lse, b, hq, s), np.where(np.isfinite(wl), wl, -1e30), rtol=1e-3, atol=1e-3)


def _paged(lens, hkv, d, bs, g, gen_kv):
    b = len(lens)
    nb = [(L + bs - 1) // bs for L in lens]
    total = sum(nb) + 2
    perm = torch.randperm(total, generator=g)
    bt = torch.zeros(b, max(nb), dtype=torch.int32)
    off = 0
    for i, n in enumerate(nb):
        bt[i, :n] = perm[off:off + n]
        off += n
    kc, vc = gen_kv((total, bs, hkv, d)), gen_kv((total, bs, hkv, d))
    return kc, vc, bt


def _gather(cache, bt, lens, bs):
    b, lmax = len(lens), max(lens)
    out = np.zeros((b, lmax) + tuple(cache.shape[2:]), cache.dtype)
    for i, L in enumerate(lens):
        pages = bt[i, :(L + bs - 1) // bs].numpy().astype(np.int64)
        out[i, :L] = cache[pages].reshape((-1,) + tuple(cache.shape[2:]))[:L]
    return out


@pytest.mark.parametrize("combined", [False, True])
def test_paged_decode_int8_kv_per_token(combined):
    """Per-token scales / offsets [B, S] (key_/value_antiquant_mode 1, or the combined [2, B, S]
    antiquant_scale with antiquant_mode 1) over a paged int8 cache, one query token per sequence."""
    g = torch.Generator().manual_seed(151)
    lens, hq, hkv, d, bs = [300, 1, 129, 64], 16, 4, 128, 64
    b = len(lens)
    kc, vc, bt = _paged(lens, hkv, d, bs, g, lambda sh: _i8(sh, g))
    smax = bt.shape[1] * bs
    ks, vs = torch.rand(b, smax, generator=g) * 0.02 + 0.005, torch.rand(b, smax, generator=g) * 0.02 + 0.005
    ko, vo = torch.rand(b, smax, generator=g) * 4 - 2, torch.rand(b, smax, generator=g) * 4 - 2
    q = torch.randn(b, 1, hq * d, generator=g).to(torch.bfloat16)
    if combined:
        kw = dict(antiquant_scale=torch.stack([ks, vs]).to(DEV), antiquant_offset=torch.stack([ko, vo]).to(DEV),
                  antiquant_mode=1)
    else:
        kw = dict(key_antiquant_scale=ks.to(DEV), key_antiquant_offset=ko.to(DEV), value_antiquant_scale=vs.to(DEV),
                  value_antiquant_offset=vo.to(DEV), key_antiquant_mode=1, value_antiquant_mode=1)
    out, lse = FIA(q.to(DEV), kc.reshape(-1, bs, hkv * d).to(DEV), vc.reshape(-1, bs, hkv * d).to(DEV),
                   block_table=bt.to(DEV), actual_seq_lengths_kv=lens, num_heads=hq, num_key_value_heads=hkv,
                   input_layout="BSH", block_size=bs, scale=1 / math.sqrt(d), softmax_lse_flag=True, **kw)
    kd = G.antiquant_kv(_gather(kc.numpy(), bt, lens, bs), ks.numpy(), ko.numpy(), 1)
    vd = G.antiquant_kv(_gather(vc.numpy(), bt, lens, bs), vs.numpy(), vo.numpy(), 1)
    want, wl = G.prefill_attention(f32np(q.reshape(b, 1, hq, d)), kd, vd, np.ones(b, np.int64), np.array(lens), 1,
                                   1 / math.sqrt(d))
    assert_close(f32np(out.reshape(b, 1, hq, d)), want)
    np.testing.assert_allclose(_lse(lse, b, hq, 1), np.where(np.isfinite(wl), wl, -1e30), rtol=1e-3, atol=1e-3)


def test_paged_multi_token_int8_kv_per_channel_bnsd_cache():
    """Legacy combined antiquant_scale [2, Hkv * D] per channel, a [blocks, Hkv, bs, D] cache, three
    query tokens per sequence (bottom-right causal)."""
    g = torch.Generator().manual_seed(152)
    lens, lq, hq, hkv, d, bs = [200, 77], 3, 8, 2, 64, 32
    b = len(lens)
    kc, vc, bt = _paged(lens, hkv, d, bs, g, lambda sh: _i8(sh, g))
    sc = torch.rand(2, hkv * d, generator=g) * 0.02 + 0.005
    q = torch.randn(b, lq, hq * d, generator=g).to(torch.bfloat16)
    out, _ = FIA(q.to(DEV), kc.permute(0, 2, 1, 3).contiguous().to(DEV), vc.permute(0, 2, 1, 3).contiguous().to(DEV),
                 block_table=bt.to(DEV), actual_seq_lengths=[lq] * b, actual_seq_lengths_kv=lens, num_heads=hq,
                 num_key_value_heads=hkv, input_layout="BSH", block_size=bs, scale=1 / math.sqrt(d), sparse_mode=3,
                 antiquant_scale=sc.to(DEV), antiquant_mode=0)
    kd = G.antiquant_kv(_gather(kc.numpy(), bt, lens, bs), sc[0].numpy(), None, 0)
    vd = G.antiquant_kv(_gather(vc.numpy(), bt, lens, bs), sc[1].numpy(), None, 0)
    want, _ = G.prefill_attention(f32np(q.reshape(b, lq, hq, d)), kd, vd, np.full(b, lq), np.array(lens), 1,
                                  1 / math.sqrt(d))
    assert_close(f32np(out.reshape(b, lq, hq, d)), want)


@pytest.mark.parametrize("per_channel", [False, True])
def test_int8_attention_out(per_channel):
    """quant_scale2 (+ quant_offset2) gives an int8 attention_out: rint(o * scale + offset) saturated."""
    g = torch.Generator().manual_seed(153)
    b, s, hq, hkv, d = 2, 70, 4, 2, 128
    q = torch.randn(b, s, hq, d, generator=g).to(torch.bfloat16)
    k = torch.randn(b, s, hkv, d, generator=g).to(torch.bfloat16)
    v = torch.randn(b, s, hkv, d, generator=g).to(torch.bfloat16)
    n = hq * d if per_channel else 1
    qs2 = torch.rand(n, generator=g) * 200 + 20
    qo2 = torch.rand(n, generator=g) * 6 - 3
    out, _ = FIA(q.to(DEV), k.to(DEV), v.to(DEV), num_heads=hq, num_key_value_heads=hkv, input_layout="BSND",
                 scale=1 / math.sqrt(d), sparse_mode=3, actual_seq_lengths=[70, 33], actual_seq_lengths_kv=[70, 33],
                 quant_scale2=qs2.to(DEV), quant_offset2=qo2.to(DEV))
    assert out.dtype == torch.int8 and out.shape == (b, s, hq, d)
    o, _ = G.prefill_attention(f32np(q), f32np(k), f32np(v), np.array([70, 33]), np.array([70, 33]), 1,
                               1 / math.sqrt(d))
    want = G.quant_attention_out(o, qs2.numpy(), qo2.numpy())
    assert_int8_close(out.cpu().numpy(), want)


def test_int8_kv_and_int8_out_paged_decode_through_the_compiled_graph():
    """int8 cache, per-channel scales and an int8 output, compiled with get_npu_backend and replayed
    from the captured graph with new lengths."""
    g = torch.Generator().manual_seed(154)
    lens, hq, hkv, d, bs = [500, 130, 7], 8, 8, 128, 128
    b = len(lens)
    kc, vc, bt = _paged(lens, hkv, d, bs, g, lambda sh: _i8(sh, g))
    ks, vs = torch.rand(hkv * d, generator=g) * 0.02, torch.rand(hkv * d, generator=g) * 0.02
    qs2 = torch.tensor([60.0])

    class M(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.register_buffer("ks", ks.to(DEV))
            self.register_buffer("vs", vs.to(DEV))
            self.register_buffer("qs2", qs2.to(DEV))

        def forward(self, q, kc, vc, bt, lens):
            # air:: takes the lengths as a device tensor (npu:: takes SymInt[])
            return torch.ops.air.npu_fused_infer_attention_score(
                q, kc, vc, block_table=bt, actual_seq_lengths_kv=lens, num_heads=hq, num_key_value_heads=hkv,
                input_layout="BSH", block_size=bs, scale=1 / math.sqrt(d), key_antiquant_scale=self.ks,
                value_antiquant_scale=self.vs, quant_scale2=self.qs2)[0]

    cfg = torchair_amd.CompilerConfig()
    cfg.mode = "reduce-overhead"
    fn = torch.compile(M(), backend=torchair_amd.get_npu_backend(compiler_config=cfg), fullgraph=True)
    kcd = kc.reshape(-1, bs, hkv * d).to(DEV)
    vcd = vc.reshape(-1, bs, hkv * d).to(DEV)
    for step_lens in (lens, [499, 1, 128]):
        q = torch.randn(b, 1, hq * d, generator=g).to(torch.bfloat16)
        out = fn(q.to(DEV), kcd, vcd, bt.to(DEV), torch.tensor(step_lens, device=DEV))
        torch.cuda.synchronize()
        kd = G.antiquant_kv(_gather(kc.numpy(), bt, step_lens, bs), ks.numpy(), None, 0)
        vd = G.antiquant_kv(_gather(vc.numpy(), bt, step_lens, bs), vs.numpy(), None, 0)
        o, _ = G.prefill_attention(f32np(q.reshape(b, 1, hq, d)), kd, vd, np.ones(b, np.int64), np.array(step_lens),
                                   1, 1 / math.sqrt(d))
        assert_int8_close(out.reshape(b, 1, hq, d).cpu().numpy(), G.quant_attention_out(o, qs2.numpy()))


@pytest.mark.parametrize("sq,mask_kw,band,bs", [(2, dict(sparse_mode=3), (1, 2147483647, 0), 64),
                                                (4, dict(sparse_mode=3), (1, 2147483647, 0), 64),
                                                (1, dict(sparse_mode=4, pre_tokens=100, next_tokens=0), (1, 100, 0), 64),
                                                (1, dict(sparse_mode=3), (1, 2147483647, 0), 16)])
def test_mla_int8_latent_several_query_tokens(sq, mask_kw, band, bs):
    """The int8 MLA latent with several query tokens per sequence (MTP / speculative decode), a window,
    or pages that are not a multiple of 32 tokens takes the general kernel with per-cache-slot scales."""
    g = torch.Generator().manual_seed(155)
    lens, h, dn, dr = [300, 65, 7], 16, 512, 64
    b = len(lens)
    nb = [(L + bs - 1) // bs for L in lens]
    total = sum(nb) + 2
    perm = torch.randperm(total, generator=g)
    bt = torch.zeros(b, max(nb), dtype=torch.int32)
    off = 0
    for i, n in enumerate(nb):
        bt[i, :n] = perm[off:off + n]
        off += n
    qn = torch.randn(b, sq, h, dn, generator=g).to(torch.bfloat16)
    qr = torch.randn(b, sq, h, dr, generator=g).to(torch.bfloat16)
    ckv = _i8((total, bs, 1, dn), g)
    cs = torch.rand(total, bs, generator=g) * 9e-3 + 1e-3
    kr = torch.randn(total, bs, 1, dr, generator=g).to(torch.bfloat16)
    scale = 1.0 / math.sqrt(192)
    out, lse = torch.ops.air.npu_fused_infer_attention_score(
        qn.to(DEV), ckv.to(DEV), ckv.to(DEV), query_rope=qr.to(DEV), key_rope=kr.to(DEV),
        key_antiquant_scale=cs.to(DEV), key_antiquant_mode=1, block_table=bt.to(DEV),
        actual_seq_lengths=torch.full((b,), sq, device=DEV), actual_seq_lengths_kv=torch.tensor(lens, device=DEV),
        num_heads=h, num_key_value_heads=1, input_layout="BSND", block_size=bs, scale=scale, softmax_lse_flag=True,
        **mask_kw)
    want, wl = G.mla_attention(f32np(qn), f32np(qr), ckv[:, :, 0].numpy(), cs.numpy(), f32np(kr[:, :, 0]), bt.numpy(),
                               [sq] * b, lens, band, scale)
    assert out.shape == (b, sq, h, dn)
    assert_close(f32np(out), want)
    np.testing.assert_allclose(_lse(lse, b, h, sq), np.where(np.isfinite(wl), wl, -1e30), rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("paged", [False, True])
def test_pse_shift(paged):
    """pse_shift [B or 1, N, S_q, S_kv] added to the scaled scores: softmax(scale * q.k + pse)."""
    g = torch.Generator().manual_seed(156)
    b, sq, hq, hkv, d = 2, 5, 8, 2, 128
    lq, lkv = [5, 3], [130, 64]
    pb = 1 if paged else b
    if paged:
        bs = 64
        kc, vc, bt = _paged(lkv, hkv, d, bs, g, lambda sh: torch.randn(sh, generator=g).to(torch.bfloat16))
        skv = bt.shape[1] * bs
    else:
        skv = 130
        k = torch.randn(b, skv, hkv, d, generator=g).to(torch.bfloat16)
        v = torch.randn(b, skv, hkv, d, generator=g).to(torch.bfloat16)
    pse = (torch.randn(pb, hq, sq, skv, generator=g) * 2).to(torch.bfloat16)
    q = torch.randn(b, sq, hq * d, generator=g).to(torch.bfloat16)
    kw = dict(actual_seq_lengths=lq, actual_seq_lengths_kv=lkv, num_heads=hq, num_key_value_heads=hkv,
              input_layout="BSH", scale=1 / math.sqrt(d), sparse_mode=3, softmax_lse_flag=True,
              pse_shift=pse.to(DEV))
    if paged:
        out, lse = FIA(q.to(DEV), kc.reshape(-1, bs, hkv * d).to(DEV), vc.reshape(-1, bs, hkv * d).to(DEV),
                       block_table=bt.to(DEV), block_size=bs, **kw)
        kd, vd = _gather(f32np(kc), bt, lkv, bs), _gather(f32np(vc), bt, lkv, bs)
    else:
        out, lse = FIA(q.to(DEV), k.reshape(b, skv, hkv * d).to(DEV), v.reshape(b, skv, hkv * d).to(DEV), **kw)
        kd, vd = f32np(k), f32np(v)
    want, wl = G.prefill_attention(f32np(q.reshape(b, sq, hq, d)), kd, vd, np.array(lq), np.array(lkv), 1,
                                   1 / math.sqrt(d), pse=f32np(pse))
    assert_close(f32np(out.reshape(b, sq, hq, d)), want)
    np.testing.assert_allclose(_lse(lse, b, hq, sq), np.where(np.isfinite(wl), wl, -1e30), rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("layout,paged", [("BSH", False), ("BNSD", False), ("BSH", True)])
def test_shared_prefix(layout, paged):
    """key_shared_prefix / value_shared_prefix: actual_shared_prefix_len rows shared by every sequence
    precede its own keys; the causal rule counts them as kv positions."""
    g = torch.Generator().manual_seed(157)
    b, sq, hq, hkv, d = 3, 4, 8, 2, 128
    lq, lkv, sp, lp = [4, 2, 4], [70, 1, 33], 96, 77
    kp = torch.randn(sp, hkv, d, generator=g).to(torch.bfloat16)
    vp = torch.randn(sp, hkv, d, generator=g).to(torch.bfloat16)
    q = torch.randn(b, sq, hq, d, generator=g).to(torch.bfloat16)
    kw = dict(actual_seq_lengths=lq, actual_seq_lengths_kv=lkv, num_heads=hq, num_key_value_heads=hkv,
              input_layout=layout, scale=1 / math.sqrt(d), sparse_mode=3, softmax_lse_flag=True,
              actual_shared_prefix_len=[lp])
    if layout == "BNSD":
        kw.update(key_shared_prefix=kp.permute(1, 0, 2)[None].contiguous().to(DEV),
                  value_shared_prefix=vp.permute(1, 0, 2)[None].contiguous().to(DEV))
        qd = q.permute(0, 2, 1, 3).contiguous().to(DEV)
    else:
        kw.update(key_shared_prefix=kp.reshape(1, sp, hkv * d).to(DEV),
                  value_shared_prefix=vp.reshape(1, sp, hkv * d).to(DEV))
        qd = q.reshape(b, sq, hq * d).to(DEV)
    if paged:
        bs = 64
        kc, vc, bt = _paged(lkv, hkv, d, bs, g, lambda sh: torch.randn(sh, generator=g).to(torch.bfloat16))
        out, lse = FIA(qd, kc.reshape(-1, bs, hkv * d).to(DEV), vc.reshape(-1, bs, hkv * d).to(DEV),
                       block_table=bt.to(DEV), block_size=bs, **kw)
        kd, vd = _gather(f32np(kc), bt, lkv, bs), _gather(f32np(vc), bt, lkv, bs)
    else:
        skv = 70
        k = torch.randn(b, skv, hkv, d, generator=g).to(torch.bfloat16)
        v = torch.randn(b, skv, hkv, d, generator=g).to(torch.bfloat16)
        if layout == "BNSD":
            out, lse = FIA(qd, k.permute(0, 2, 1, 3).contiguous().to(DEV), v.permute(0, 2, 1, 3).contiguous().to(DEV),
                           **kw)
        else:
            out, lse = FIA(qd, k.reshape(b, skv, hkv * d).to(DEV), v.reshape(b, skv, hkv * d).to(DEV), **kw)
        kd, vd = f32np(k), f32np(v)
    kk, vv, ll = G.with_shared_prefix(kd, vd, np.array(lkv), f32np(kp), f32np(vp), lp)
    want, wl = G.prefill_attention(f32np(q), kk, vv, np.array(lq), ll, 1, 1 / math.sqrt(d))
    got = out.cpu() if layout != "BNSD" else out.cpu().permute(0, 2, 1, 3)
    assert_close(f32np(got.reshape(b, sq, hq, d)), want)
    np.testing.assert_allclose(_lse(lse, b, hq, sq), np.where(np.isfinite(wl), wl, -1e30), rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("paged", [False, True])
def test_shared_prefix_int8_cache(paged):
    """A bf16 shared prefix ahead of int8 own keys/values: the prefix rows are read as they are, the
    own rows dequantised with scales indexed by the sequence's own positions (per token on the paged
    cache, per channel on the dense one)."""
    g = torch.Generator().manual_seed(158)
    b, sq, hq, hkv, d = 2, 3, 8, 2, 128
    lq, lkv, sp, lp = [3, 1], [90, 17], 40, 33
    kp = torch.randn(sp, hkv, d, generator=g).to(torch.bfloat16)
    vp = torch.randn(sp, hkv, d, generator=g).to(torch.bfloat16)
    q = torch.randn(b, sq, hq, d, generator=g).to(torch.bfloat16)
    kw = dict(actual_seq_lengths=lq, actual_seq_lengths_kv=lkv, num_heads=hq, num_key_value_heads=hkv,
              input_layout="BSH", scale=1 / math.sqrt(d), sparse_mode=3, softmax_lse_flag=True,
              actual_shared_prefix_len=[lp], key_shared_prefix=kp.reshape(1, sp, hkv * d).to(DEV),
              value_shared_prefix=vp.reshape(1, sp, hkv * d).to(DEV))
    if paged:
        bs = 32
        kc, vc, bt = _paged(lkv, hkv, d, bs, g, lambda sh: _i8(sh, g))
        smax = bt.shape[1] * bs
        ks, vs = torch.rand(b, smax, generator=g) * 0.02 + 0.005, torch.rand(b, smax, generator=g) * 0.02 + 0.005
        out, lse = FIA(q.reshape(b, sq, hq * d).to(DEV), kc.reshape(-1, bs, hkv * d).to(DEV),
                       vc.reshape(-1, bs, hkv * d).to(DEV), block_table=bt.to(DEV), block_size=bs,
                       key_antiquant_scale=ks.to(DEV), value_antiquant_scale=vs.to(DEV), key_antiquant_mode=1,
                       value_antiquant_mode=1, **kw)
        kd = G.antiquant_kv(_gather(kc.numpy(), bt, lkv, bs), ks.numpy(), None, 1)
        vd = G.antiquant_kv(_gather(vc.numpy(), bt, lkv, bs), vs.numpy(), None, 1)
    else:
        skv = 90
        k, v = _i8((b, skv, hkv, d), g), _i8((b, skv, hkv, d), g)
        ks, vs = torch.rand(hkv * d, generator=g) * 0.02 + 0.005, torch.rand(hkv * d, generator=g) * 0.02 + 0.005
        out, lse = FIA(q.reshape(b, sq, hq * d).to(DEV), k.reshape(b, skv, hkv * d).to(DEV),
                       v.reshape(b, skv, hkv * d).to(DEV), key_antiquant_scale=ks.to(DEV),
                       value_antiquant_scale=vs.to(DEV), **kw)
        kd = G.antiquant_kv(k.numpy(), ks.numpy(), None, 0)
        vd = G.antiquant_kv(v.numpy(), vs.numpy(), None, 0)
    kk, vv, ll = G.with_shared_prefix(kd, vd, np.array(lkv), f32np(kp), f32np(vp), lp)
    want, wl = G.prefill_attention(f32np(q), kk, vv, np.array(lq), ll, 1, 1 / math.sqrt(d))
    assert_close(f32np(out.reshape(b, sq, hq, d)), want)
    np.testing.assert_allclose(_lse(lse, b, hq, sq), np.where(np.isfinite(wl), wl, -1e30), rtol=1e-3, atol=1e-3)


def _u64(x):
    """An fp32 value in the low 32 bits of a UINT64 tensor (the prototype's dequant_scale format)."""
    return torch.tensor([int(np.array([x], np.float32).view(np.uint32)[0])], dtype=torch.int64)


@pytest.mark.parametrize("paged,scale_form,out8", [(False, "f32", False), (False, "u64", True), (True, "u64", False)])
def test_int8_query(paged, scale_form, out8):
    """An int8 query, key and value with dequant_scale1 / quant_scale1 / dequant_scale2 (per tensor; the
    dequant scales as fp32 or as UINT64 carrying an fp32): the oracle's two-pass convention, fp16 out
    (or int8 with quant_scale2). Tolerance: a P8 that rounds the other way between the device's and
    numpy's exp moves an output by at most 127 * dequant_scale2 / l <= 0.0127, hence atol 2e-2."""
    g = torch.Generator().manual_seed(159)
    b, sq, hq, hkv, d = 2, 4, 8, 2, 128
    lq, lkv = [4, 1], ([300, 77] if paged else [96, 50])
    d1, q1, d2 = 4e-4, 127.0, 1e-4
    q = _i8((b, sq, hq, d), g)
    kw = dict(actual_seq_lengths=lq, actual_seq_lengths_kv=lkv, num_heads=hq, num_key_value_heads=hkv,
              input_layout="BSH", scale=1 / math.sqrt(d), sparse_mode=3, softmax_lse_flag=True,
              quant_scale1=torch.tensor([q1], device=DEV))
    if scale_form == "u64":
        kw.update(dequant_scale1=_u64(d1).to(DEV), dequant_scale2=_u64(d2).to(DEV))
    else:
        kw.update(dequant_scale1=torch.tensor([d1], device=DEV), dequant_scale2=torch.tensor([d2], device=DEV))
    if out8:
        kw["quant_scale2"] = torch.tensor([50.0], device=DEV)
    if paged:
        bs = 64
        kc, vc, bt = _paged(lkv, hkv, d, bs, g, lambda sh: _i8(sh, g))
        out, lse = FIA(q.reshape(b, sq, hq * d).to(DEV), kc.reshape(-1, bs, hkv * d).to(DEV),
                       vc.reshape(-1, bs, hkv * d).to(DEV), block_table=bt.to(DEV), block_size=bs, **kw)
        kd, vd = _gather(kc.numpy(), bt, lkv, bs), _gather(vc.numpy(), bt, lkv, bs)
    else:
        skv = 96
        k, v = _i8((b, skv, hkv, d), g), _i8((b, skv, hkv, d), g)
        out, lse = FIA(q.reshape(b, sq, hq * d).to(DEV), k.reshape(b, skv, hkv * d).to(DEV),
                       v.reshape(b, skv, hkv * d).to(DEV), **kw)
        kd, vd = k.numpy(), v.numpy()
    want, wl = G.quant_query_attention(q.numpy(), kd, vd, d1, q1, d2, lq, lkv, (1, 2147483647, 0), 1 / math.sqrt(d))
    if out8:
        assert out.dtype == torch.int8
        got = out.reshape(b, sq, hq, d).cpu().numpy().astype(np.int32)
        exp8 = G.quant_attention_out(want, [50.0]).astype(np.int32)
        assert np.abs(got - exp8).max() <= 1
    else:
        assert out.dtype == torch.float16
        assert_close(f32np(out.reshape(b, sq, hq, d)), want, atol=2e-2)
    np.testing.assert_allclose(_lse(lse, b, hq, sq), np.where(np.isfinite(wl), wl, -1e30), rtol=1e-3, atol=1e-3)


def test_int8_query_argument_errors():
    q = torch.zeros(1, 1, 128, dtype=torch.int8, device=DEV)
    one = torch.ones(1, device=DEV)
    with pytest.raises(RuntimeError, match="dequant_scale1"):
        FIA(q, q, q, num_heads=1, dequant_scale1=one)
    x = torch.zeros(1, 1, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="int8 query"):
        FIA(x, x, x, num_heads=1, dequant_scale1=one, quant_scale1=one, dequant_scale2=one)
