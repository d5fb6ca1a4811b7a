"""int8 key / value caches with per-channel antiquant scales on the one-token paged decode kernel
(tai_fia_paged_decode_kv8): the covered pages are widened to 16-bit values, the query takes the key
scale and the merge the value scale. Compared with the oracle on the dequantised caches
(oracle/golden.py antiquant_kv rule: x * scale per channel), including an empty sequence, fp16 and head
dims 64, 128 and 256; a cache with offsets stays on the general kernel."""
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
FIA = torch.ops.npu.npu_fused_infer_attention_score


def _case(d, hq, hkv, dtype, offsets, monkeypatch):
    g = torch.Generator().manual_seed(7 * d + hq)
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
    kc = torch.randint(-128, 128, (total, bs, hkv, d), generator=g, dtype=torch.int8)
    vc = torch.randint(-128, 128, (total, bs, hkv, d), generator=g, dtype=torch.int8)
    ks = torch.rand(hkv * d, generator=g) * 0.02 + 0.005
    vs = torch.rand(hkv * d, generator=g) * 0.02 + 0.005
    ko = (torch.randint(-4, 5, (hkv * d,), generator=g).float()) if offsets else None
    scale = 1 / math.sqrt(d)
    called = []
    real = _lib.call
    monkeypatch.setattr(_lib, "call", lambda name, *a: (called.append(name), real(name, *a))[1])
    print("case", dict(d=d, hq=hq, hkv=hkv, dtype=str(dtype), offsets=offsets), flush=True)
    kw = dict(key_antiquant_scale=ks.to(DEV), value_antiquant_scale=vs.to(DEV))
    if ko is not None:
        kw["key_antiquant_offset"] = ko.to(DEV)
    out, lse = FIA(q.reshape(b, 1, hq * d).to(DEV), kc.reshape(total, bs, hkv * d).to(DEV),
                   vc.reshape(total, bs, hkv * d).to(DEV), actual_seq_lengths_kv=lk, block_table=bt.to(DEV),
                   block_size=bs, num_heads=hq, num_key_value_heads=hkv, input_layout="BSH", scale=scale,
                   softmax_lse_flag=True, **kw)
    torch.cuda.synchronize()
    kd = (kc.numpy().astype(np.float32) + (0 if ko is None else ko.numpy().reshape(hkv, d))) * ks.numpy().reshape(hkv, d)
    vd = vc.numpy().astype(np.float32) * vs.numpy().reshape(hkv, d)
    want, wl = G.paged_prefill_attention(f32np(q), kd.astype(np.float32), vd.astype(np.float32), bt.numpy(), [1] * b,
                                         lk, (0, 2**31 - 1, 2**31 - 1), scale)
    got = f32np(out.cpu()).reshape(b, 1, hq, d)
    assert_close(got[1:], want[1:])
    assert np.all(got[0] == 0)
    # the 16-bit MFMA takes q * key scale rounded to the query dtype: scores (and lse) carry a relative
    # error of about 2^-9, against the oracle's fp32 dequantisation
    np.testing.assert_allclose(lse.cpu().numpy().reshape(b, hq)[1:], wl[1:, :, 0], rtol=1e-2, atol=1e-2)
    return called


@pytest.mark.parametrize("d,hq,hkv,dtype", [(128, 32, 8, torch.bfloat16), (64, 8, 1, torch.float16),
                                            (256, 16, 4, torch.bfloat16)])
def test_paged_decode_int8_cache(d, hq, hkv, dtype, monkeypatch):
    called = _case(d, hq, hkv, dtype, False, monkeypatch)
    assert "tai_fia_paged_decode_kv8" in called, called


def test_paged_decode_int8_cache_with_offsets_takes_the_general_kernel(monkeypatch):
    called = _case(128, 16, 4, torch.bfloat16, True, monkeypatch)
    assert "tai_fia_general" in called and "tai_fia_paged_decode_kv8" not in called, called
