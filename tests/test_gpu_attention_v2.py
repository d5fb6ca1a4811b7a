"""GPU: npu_fused_infer_attention_score_v2 (air:: with tensor lengths, npu:: with list lengths) is the
v1 operator under renamed arguments (the reference lowers both to one FusedInferAttentionScore node,
python/torchair/ops/_npu_fused_infer_attention_score_v2.py:166-181), so each case must equal the v1
call with the mapped arguments bit for bit."""
import math

import pytest
import torch

import torchair_amd  # noqa: F401

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


@pytest.mark.parametrize("arg", ["learnable_sink", "dequant_scale_query", "quant_scale_p"])
def test_v2_refuses_what_it_does_not_serve(arg):
    q = torch.randn(1, 8, 4 * 64, device=DEV).to(torch.bfloat16)
    with pytest.raises(RuntimeError, match=arg):
        V2(q, q, q, num_query_heads=4, input_layout="BSH", **{arg: torch.ones(4, device=DEV)})
