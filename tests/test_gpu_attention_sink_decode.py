"""learnable_sink on the one-token paged decode kernel (tai_fia_paged_decode_sink): the v2 op with a sink
and no other general-kernel feature runs the decode kernel, whose merge takes each head's sink logit into
the row's max and denominator. Compared with the oracle (oracle/golden.py paged_prefill_attention with
sink), including a head whose sink is -inf (no effect), an empty sequence (zeros, lse = the sink) and
fp16, at head dims 64, 128 and 256."""
import math

import numpy as np
import pytest
import torch

import torchair_amd  # noqa: F401
from oracle import golden as G
from tests.helpers import assert_close, f32np
from torchair_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"
V2 = torch.ops.npu.npu_fused_infer_attention_score_v2


@pytest.mark.parametrize("d,hq,hkv,dtype", [(128, 32, 8, torch.bfloat16), (64, 8, 1, torch.float16),
                                            (256, 16, 4, torch.bfloat16)])
def test_paged_decode_with_sink(d, hq, hkv, dtype, monkeypatch):
    g = torch.Generator().manual_seed(d + hq)
    b, bs = 5, 64
    lk = [0, 1, 77, 300, 1000]
    nb = [max(1, (x + bs - 1) // bs) for x in lk]
    total = sum(nb) + 1
    perm = torch.randperm(total, generator=g)
    bt = torch.zeros(b, max(nb), dtype=torch.int32)
    o = 0
    for i, n in enumerate(nb):
        bt[i, :n] = perm[o:o + n]
        o += n
    q = torch.randn(b, 1, hq, d, generator=g).to(dtype)
    kc = torch.randn(total, bs, hkv, d, generator=g).to(dtype)
    vc = torch.randn(total, bs, hkv, d, generator=g).to(dtype)
    sink = (torch.randn(hq, generator=g) * 2).to(dtype)
    sink[1] = float("-inf")
    scale = 1 / math.sqrt(d)
    called = []
    real = _lib.call
    monkeypatch.setattr(_lib, "call", lambda name, *a: (called.append(name), real(name, *a))[1])
    print("case", dict(d=d, hq=hq, hkv=hkv, dtype=str(dtype), lk=lk), flush=True)
    out, lse = V2(q.reshape(b, 1, hq * d).to(DEV), kc.reshape(total, bs, hkv * d).to(DEV),
                  vc.reshape(total, bs, hkv * d).to(DEV), actual_seq_kvlen=lk, block_table=bt.to(DEV), block_size=bs,
                  num_query_heads=hq, num_key_value_heads=hkv, input_layout="BSH", softmax_scale=scale,
                  learnable_sink=sink.to(DEV), return_softmax_lse=True)
    torch.cuda.synchronize()
    assert "tai_fia_paged_decode_sink" in called, called
    want, wl = G.paged_prefill_attention(f32np(q), f32np(kc), f32np(vc), bt.numpy(), [1] * b, lk, (0, 2**31 - 1, 2**31 - 1),
                                         scale, sink=f32np(sink))
    got = f32np(out.cpu()).reshape(b, 1, hq, d)
    assert_close(got[1:], want[1:])
    assert np.all(got[0] == 0)  # no keys: the sink alone, no value rows
    lg = lse.cpu().numpy().reshape(b, hq)
    np.testing.assert_allclose(lg[1:], wl[1:, :, 0], rtol=1e-3, atol=1e-3)
    s = f32np(sink)
    np.testing.assert_allclose(lg[0], s, rtol=1e-3, atol=1e-3)  # lse of an empty row is its sink (-inf for none)
