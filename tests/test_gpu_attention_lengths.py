"""GPU: sequence lengths read on the device are clamped to the extent the inputs hold.

A length past the cache extent a block-table row can address (max_blocks * block_size), or past
the dense S_q / S_kv, must not index past its block-table row into other sequences' blocks or past
the tensors. The kernels clamp it; each case checks that the output equals, bit for bit, the output
of the same call with the lengths clamped on the host."""
import math

import pytest
import torch

import torchair_amd  # noqa: F401
from tests.test_gpu_attention import _mla_case, _paged_case, _paged_seq_case

pytestmark = pytest.mark.gpu
DEV = "cuda"
FIA = torch.ops.air.npu_fused_infer_attention_score


def _same(a, b):
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_paged_decode_length_past_block_table_is_clamped():
    hq, hkv, d, bs = 8, 2, 128, 64
    q, k4, v4, bt, _ = _paged_case([77, 300, 130], hq, hkv, d, bs, 140)
    cap = bt.shape[1] * bs
    kc = k4.reshape(k4.shape[0], bs, hkv * d).to(DEV)
    vc = v4.reshape(v4.shape[0], bs, hkv * d).to(DEV)
    kw = dict(block_table=bt.to(DEV), num_heads=hq, num_key_value_heads=hkv, input_layout="BSH", block_size=bs,
              scale=1.0 / math.sqrt(d), softmax_lse_flag=True)
    qd = q.reshape(3, 1, hq * d).to(DEV)
    over = FIA(qd, kc, vc, actual_seq_lengths_kv=torch.tensor([77, 10 ** 9, -5], device=DEV), **kw)
    clamped = FIA(qd, kc, vc, actual_seq_lengths_kv=torch.tensor([77, cap, 0], device=DEV), **kw)
    _same(over, clamped)


@pytest.mark.parametrize("bs", [64, 16])
def test_paged_prefill_lengths_past_extent_are_clamped(bs):
    """bs 64 takes the prefill kernel, bs 16 the general kernel."""
    lq, lkv = [3, 2], [200, 77]
    hq, hkv, d = 8, 2, 128
    q, k4, v4, bt = _paged_seq_case(lq, lkv, hq, hkv, d, bs, 141)
    cap = bt.shape[1] * bs
    kc = k4.reshape(k4.shape[0], bs, hkv * d).to(DEV)
    vc = v4.reshape(v4.shape[0], bs, hkv * d).to(DEV)
    qa = q.reshape(2, 3, hq * d).to(DEV)
    kw = dict(block_table=bt.to(DEV), num_heads=hq, num_key_value_heads=hkv, input_layout="BSH", block_size=bs,
              scale=1.0 / math.sqrt(d), softmax_lse_flag=True, sparse_mode=3)
    over = FIA(qa, kc, vc, actual_seq_lengths=torch.tensor([99, 2], device=DEV),
               actual_seq_lengths_kv=torch.tensor([200, 10 ** 7], device=DEV), **kw)
    clamped = FIA(qa, kc, vc, actual_seq_lengths=torch.tensor([3, 2], device=DEV),
                  actual_seq_lengths_kv=torch.tensor([200, cap], device=DEV), **kw)
    _same(over, clamped)


def test_dense_prefill_lengths_past_extent_are_clamped():
    gen = torch.Generator(device=DEV).manual_seed(142)
    b, s, hq, hkv, d = 2, 96, 4, 2, 128
    q = torch.randn(b, s, hq * d, generator=gen, device=DEV).to(torch.bfloat16)
    k = torch.randn(b, s, hkv * d, generator=gen, device=DEV).to(torch.bfloat16)
    v = torch.randn(b, s, hkv * d, generator=gen, device=DEV).to(torch.bfloat16)
    kw = dict(num_heads=hq, num_key_value_heads=hkv, input_layout="BSH", scale=1.0 / math.sqrt(d), sparse_mode=3,
              softmax_lse_flag=True)
    over = FIA(q, k, v, actual_seq_lengths=torch.tensor([500, 40], device=DEV),
               actual_seq_lengths_kv=torch.tensor([1000, 60], device=DEV), **kw)
    clamped = FIA(q, k, v, actual_seq_lengths=torch.tensor([96, 40], device=DEV),
                  actual_seq_lengths_kv=torch.tensor([96, 60], device=DEV), **kw)
    _same(over, clamped)


def test_mla_length_past_block_table_is_clamped():
    h, bs = 16, 64
    qn, qr, ckv, cs, kr, bt = _mla_case([300, 65, 1], h, bs, 143)
    cap = bt.shape[1] * bs

    def run(lens):
        return FIA(qn.to(DEV), ckv.to(DEV), ckv.to(DEV), query_rope=qr.to(DEV), key_rope=kr.to(DEV),
                   key_antiquant_scale=cs.to(DEV), key_antiquant_mode=1, block_table=bt.to(DEV),
                   actual_seq_lengths_kv=torch.tensor(lens, device=DEV), num_heads=h, num_key_value_heads=1,
                   input_layout="BSND", block_size=bs, scale=1.0 / math.sqrt(192), softmax_lse_flag=True)

    _same(run([300, 10 ** 8, 1]), run([300, cap, 1]))
