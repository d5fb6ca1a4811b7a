"""GPU: npu_fused_infer_attention_score_v2 (air:: with tensor lengths, npu:: with list lengths) is the
v1 operator under renamed arguments (the reference lowers both to one FusedInferAttentionScore node,
python/torchair/ops/_npu_fused_infer_attention_score_v2.py:166-181), so each case must equal the v1
call with the mapped arguments bit for bit; learnable_sink, which only v2 takes, is checked against the
oracle."""
import math

import numpy as np
import pytest
import torch

import torchair_amd  # noqa: F401
from oracle import golden as G
from tests.helpers import assert_close, f32np

pytestmark = pytest.mark.gpu
DEV = "cuda"
V1, V2 = torch.ops.npu.npu_fused_infer_attention_score, torch.ops.air.npu_fused_infer_attention_score_v2
V2N = torch.ops.npu.npu_fused_infer_attention_score_v2


def _eq(a, b):
    assert a.dtype == b.dtype and a.shape == b.shape
    assert torch.equal(torch.nan_to_num(a.float(), 7.0), torch.nan_to_num(b.float(), 7.0))


def test_v2_causal_prefill_with_lse():
    g = torch.Generator().manual_seed(90)
    b, s, hq, hkv, d = 2, 200, 8, 2, 128
    q = torch.randn(b, s, hq * d, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(b, s, hkv * d, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(b, s, hkv * d, generator=g).to(torch.bfloat16).to(DEV)
    lens = [200, 77]
    o1, l1 = V1(q, k, v, actual_seq_lengths=lens, actual_seq_lengths_kv=lens, num_heads=hq, num_key_value_heads=hkv,
                input_layout="BSH", scale=1 / math.sqrt(d), sparse_mode=3, softmax_lse_flag=True)
    lt = torch.tensor(lens, device=DEV)
    o2, l2 = V2(q, k, v, actual_seq_qlen=lt, actual_seq_kvlen=lt, num_query_heads=hq, num_key_value_heads=hkv,
                input_layout="BSH", softmax_scale=1 / math.sqrt(d), sparse_mode=3, return_softmax_lse=True)
    o3, l3 = V2N(q, k, v, actual_seq_qlen=lens, actual_seq_kvlen=lens, num_query_heads=hq, num_key_value_heads=hkv,
                 input_layout="BSH", softmax_scale=1 / math.sqrt(d), sparse_mode=3, return_softmax_lse=True)
    for o, l in ((o2, l2), (o3, l3)):
        _eq(o, o1)
        _eq(l, l1)


def test_v2_paged_int8_cache_and_int8_out():
    g = torch.Generator().manual_seed(91)
    b, hq, hkv, d, bs = 4, 16, 2, 128, 64
    lens = [300, 64, 1, 190]
    nb = [(L + bs - 1) // bs for L in lens]
    total = sum(nb) + 1
    bt = torch.zeros(b, max(nb), dtype=torch.int32)
    perm = torch.randperm(total, generator=g)
    o = 0
    for i, n in enumerate(nb):
        bt[i, :n] = perm[o:o + n]
        o += n
    kc = torch.randint(-128, 128, (total, bs, hkv * d), generator=g, dtype=torch.int8).to(DEV)
    vc = torch.randint(-128, 128, (total, bs, hkv * d), generator=g, dtype=torch.int8).to(DEV)
    ks = (torch.rand(hkv * d, generator=g) * 0.02 + 0.005).to(DEV)
    vs = (torch.rand(hkv * d, generator=g) * 0.02 + 0.005).to(DEV)
    qs2 = (torch.rand(1, generator=g) * 20 + 5).to(DEV)
    q = torch.randn(b, 1, hq * d, generator=g).to(torch.bfloat16).to(DEV)
    o1, _ = V1(q, kc, vc, actual_seq_lengths_kv=lens, block_table=bt.to(DEV), block_size=bs, num_heads=hq,
               num_key_value_heads=hkv, input_layout="BSH", scale=1 / math.sqrt(d), key_antiquant_scale=ks,
               value_antiquant_scale=vs, quant_scale2=qs2)
    o2, _ = V2N(q, kc, vc, actual_seq_kvlen=lens, block_table=bt.to(DEV), block_size=bs, num_query_heads=hq,
                num_key_value_heads=hkv, input_layout="BSH", softmax_scale=1 / math.sqrt(d), dequant_scale_key=ks,
                dequant_scale_value=vs, quant_scale_out=qs2)
    assert o1.dtype == torch.int8
    _eq(o2, o1)


@pytest.mark.parametrize("arg", ["dequant_scale_query", "quant_scale_p"])
def test_v2_refuses_what_it_does_not_serve(arg):
    q = torch.randn(1, 8, 4 * 64, device=DEV).to(torch.bfloat16)
    with pytest.raises(RuntimeError, match=arg):
        V2(q, q, q, num_query_heads=4, input_layout="BSH", **{arg: torch.ones(4, device=DEV)})


def test_v2_learnable_sink_needs_one_logit_per_head():
    q = torch.randn(1, 8, 4 * 64, device=DEV).to(torch.bfloat16)
    with pytest.raises(RuntimeError, match="learnable_sink"):
        V2(q, q, q, num_query_heads=4, input_layout="BSH", learnable_sink=torch.ones(3, device=DEV))


_BIG = 2147483647


@pytest.mark.parametrize("layout", ["BSH", "BNSD"])
def test_v2_learnable_sink_dense_prefill(layout):
    """learnable_sink (bf16, one logit per query head) joins the softmax denominator: dense causal
    prefill on the general kernel against the oracle."""
    g = torch.Generator().manual_seed(180)
    b, s, hq, hkv, d = 2, 40, 8, 2, 128
    lens = [40, 17]
    q = torch.randn(b, s, hq, d, generator=g).to(torch.bfloat16)
    k = torch.randn(b, s, hkv, d, generator=g).to(torch.bfloat16)
    v = torch.randn(b, s, hkv, d, generator=g).to(torch.bfloat16)
    sink = (torch.randn(hq, generator=g) * 2).to(torch.bfloat16)
    if layout == "BSH":
        qd, kd, vd = (t.reshape(b, s, -1).to(DEV) for t in (q, k, v))
    else:
        qd, kd, vd = (t.permute(0, 2, 1, 3).contiguous().to(DEV) for t in (q, k, v))
    out, lse = torch.ops.npu.npu_fused_infer_attention_score_v2(
        qd, kd, vd, actual_seq_qlen=lens, actual_seq_kvlen=lens, num_query_heads=hq, num_key_value_heads=hkv,
        input_layout=layout, softmax_scale=1 / math.sqrt(d), sparse_mode=3, return_softmax_lse=True,
        learnable_sink=sink.to(DEV))
    want, wl = G.prefill_attention(f32np(q), f32np(k), f32np(v), np.array(lens), np.array(lens), 1, 1 / math.sqrt(d),
                                   sink=f32np(sink))
    got = out.cpu() if layout == "BSH" else out.cpu().permute(0, 2, 1, 3)
    assert_close(f32np(got.reshape(b, s, hq, d)), want)
    np.testing.assert_allclose(np.where(np.isfinite(wl), wl, -1e30),
                               np.where(np.isfinite(lse.cpu().numpy()), lse.cpu().numpy(), -1e30).reshape(b, hq, s),
                               rtol=1e-3, atol=1e-3)


def test_v2_learnable_sink_paged_decode_and_packed():
    """The sink on a paged cache, one query token per sequence (TND, list ends 1..B), and on packed
    chunked-prefill queries."""
    g = torch.Generator().manual_seed(181)
    lk, hq, hkv, d, bs = [300, 1, 129, 64], 16, 4, 128, 64
    bn = len(lk)
    nb = [(L + bs - 1) // bs for L in lk]
    total = sum(nb) + 2
    perm = torch.randperm(total, generator=g)
    bt = torch.zeros(bn, max(nb), dtype=torch.int32)
    off = 0
    for i, n in enumerate(nb):
        bt[i, :n] = perm[off:off + n]
        off += n
    kc = torch.randn(total, bs, hkv, d, generator=g).to(torch.bfloat16)
    vc = torch.randn(total, bs, hkv, d, generator=g).to(torch.bfloat16)
    sink = (torch.randn(hq, generator=g) * 2).to(torch.bfloat16)
    for lq in ([1, 1, 1, 1], [2, 1, 5, 3]):
        t = sum(lq)
        q = torch.randn(t, hq, d, generator=g).to(torch.bfloat16)
        cq = np.cumsum(lq).tolist()
        out, _ = torch.ops.npu.npu_fused_infer_attention_score_v2(
            q.to(DEV), kc.reshape(-1, bs, hkv * d).to(DEV), vc.reshape(-1, bs, hkv * d).to(DEV),
            block_table=bt.to(DEV), actual_seq_qlen=cq, actual_seq_kvlen=lk, num_query_heads=hq,
            num_key_value_heads=hkv, input_layout="TND", block_size=bs, softmax_scale=1 / math.sqrt(d), sparse_mode=3,
            learnable_sink=sink.to(DEV))
        qb = G.unpack_tnd(f32np(q), cq, max(lq))
        o, _ = G.paged_prefill_attention(qb, f32np(kc), f32np(vc), bt.numpy(), lq, lk, (1, _BIG, 0),
                                         1 / math.sqrt(d), sink=f32np(sink))
        assert_close(f32np(out), G.pack_tnd(o, lq))


def test_v2_learnable_sink_mla_bf16_latent():
    """The sink on the MLA general path (bf16 latent, two query tokens)."""
    g = torch.Generator().manual_seed(182)
    lens, h, dn, dr, bs, sq = [70, 33], 16, 512, 64, 32, 2
    b = len(lens)
    nb = [(L + bs - 1) // bs for L in lens]
    total = sum(nb) + 1
    perm = torch.randperm(total, generator=g)
    bt = torch.zeros(b, max(nb), dtype=torch.int32)
    off = 0
    for i, n in enumerate(nb):
        bt[i, :n] = perm[off:off + n]
        off += n
    qn = torch.randn(b, sq, h, dn, generator=g).to(torch.bfloat16)
    qr = torch.randn(b, sq, h, dr, generator=g).to(torch.bfloat16)
    ckv = (torch.randn(total, bs, 1, dn, generator=g) * 0.5).to(torch.bfloat16)
    kr = torch.randn(total, bs, 1, dr, generator=g).to(torch.bfloat16)
    sink = (torch.randn(h, generator=g) * 2).to(torch.bfloat16)
    scale = 1.0 / math.sqrt(192)
    out, _ = torch.ops.npu.npu_fused_infer_attention_score_v2(
        qn.to(DEV), ckv.to(DEV), ckv.to(DEV), query_rope=qr.to(DEV), key_rope=kr.to(DEV), block_table=bt.to(DEV),
        actual_seq_qlen=[sq] * b, actual_seq_kvlen=lens, num_query_heads=h, num_key_value_heads=1,
        input_layout="BSND", block_size=bs, softmax_scale=scale, sparse_mode=3, learnable_sink=sink.to(DEV))
    want, _ = G.mla_attention(f32np(qn), f32np(qr), f32np(ckv[:, :, 0]), None, f32np(kr[:, :, 0]), bt.numpy(),
                              [sq] * b, lens, (1, _BIG, 0), scale, sink=f32np(sink))
    assert_close(f32np(out), want)
