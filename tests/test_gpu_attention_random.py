"""Seeded random configurations of npu_fused_infer_attention_score_v2 against the oracle: layout
(BSH / BSND / BNSD), dense or paged K/V (page sizes that are and are not multiples of 32), bf16 or
int8 caches (per-channel antiquant), causal / band / no mask, learnable_sink, GQA ratios, head dims and
int8 attention_out, each with ragged sequence lengths. The combinations reach every kernel of the
attention path (decode, prefill, general)."""
import math

import numpy as np
import pytest
import torch

import torchair_amd  # noqa: F401
from oracle import golden as G
from tests.helpers import assert_close, f32np

pytestmark = pytest.mark.gpu
DEV = "cuda"
V2 = torch.ops.npu.npu_fused_infer_attention_score_v2
BIG = 2147483647


def _to_layout(t, layout):
    """[B, S, N, D] -> the layout's tensor."""
    if layout == "BSH":
        return t.reshape(t.shape[0], t.shape[1], -1)
    if layout == "BNSD":
        return t.permute(0, 2, 1, 3).contiguous()
    return t.contiguous()


def _from_layout(t, layout, n):
    if layout == "BSH":
        return t.reshape(t.shape[0], t.shape[1], n, -1)
    if layout == "BNSD":
        return t.permute(0, 2, 1, 3)
    return t


@pytest.mark.parametrize("seed", range(24))
def test_random_attention_configuration(seed):
    rng = np.random.default_rng(2000 + seed)
    g = torch.Generator().manual_seed(2000 + seed)
    b = int(rng.integers(1, 5))
    hkv = int(rng.choice([1, 2, 4]))
    hq = hkv * int(rng.choice([1, 2, 4, 8]))
    d = int(rng.choice([64, 128]))
    layout = str(rng.choice(["BSH", "BSND", "BNSD"]))
    paged = bool(rng.integers(0, 2))
    kv8 = bool(rng.integers(0, 2))
    sink_on = bool(rng.integers(0, 2))
    out8 = bool(rng.integers(0, 3) == 0)
    if rng.integers(0, 3) == 0:  # a third of the cases without the general kernel's features (fast kernels)
        kv8 = sink_on = out8 = False
    mode = int(rng.choice([0, 3, 4]))
    sq = int(rng.choice([1, 1, 3, 17]))
    lq = [int(rng.integers(1, sq + 1)) for _ in range(b)]
    lk = [int(x + rng.integers(0, 200)) for x in lq]
    pre, nxt = int(rng.integers(5, 60)), int(rng.integers(0, 3))
    kw = dict(sparse_mode=mode)
    if mode == 4:
        kw.update(pre_tokens=pre, next_tokens=nxt)
    band = {0: (0, BIG, BIG), 3: (1, BIG, 0), 4: (1, pre, nxt)}[mode]
    scale = 1 / math.sqrt(d)
    q = torch.randn(b, sq, hq, d, generator=g).to(torch.bfloat16)
    sink = (torch.randn(hq, generator=g) * 2).to(torch.bfloat16) if sink_on else None
    ks = vs = None
    if kv8:
        ks = torch.rand(hkv * d, generator=g) * 0.02 + 0.005
        vs = torch.rand(hkv * d, generator=g) * 0.02 + 0.005

    def make(shape):
        if kv8:
            return torch.randint(-128, 128, shape, generator=g, dtype=torch.int8)
        return torch.randn(shape, generator=g).to(torch.bfloat16)

    def deq(t, sc):  # [..., Hkv, D] host tensor -> fp32 numpy (dequantised when int8)
        if not kv8:
            return f32np(t)
        x = t.numpy().astype(np.float32)
        return (x * sc.numpy().reshape(hkv, d)).astype(np.float32)

    if paged:
        bs = int(rng.choice([16, 32, 64, 128]))
        nb = [(L + bs - 1) // bs for L in lk]
        total = sum(nb) + 2
        perm = torch.randperm(total, generator=g)
        bt = torch.zeros(b, max(nb), dtype=torch.int32)
        off = 0
        for i, n in enumerate(nb):
            bt[i, :n] = perm[off:off + n]
            off += n
        kc, vc = make((total, bs, hkv, d)), make((total, bs, hkv, d))
        kd = kc.reshape(total, bs, hkv * d).to(DEV)
        vd = vc.reshape(total, bs, hkv * d).to(DEV)
        qd = _to_layout(q, layout).to(DEV)
        if layout != "BSH":
            kw["input_layout"] = layout
        extra = dict(block_table=bt.to(DEV), block_size=bs)
        want, wl = G.paged_prefill_attention(f32np(q), deq(kc, ks), deq(vc, vs), bt.numpy(), lq, lk, band, scale,
                                             sink=None if sink is None else f32np(sink))
    else:
        skv = max(lk)
        k, v = make((b, skv, hkv, d)), make((b, skv, hkv, d))
        qd, kd, vd = (_to_layout(t, layout).to(DEV) for t in (q, k, v))
        extra = {}
        want, wl = G.prefill_attention(f32np(q), deq(k, ks), deq(v, vs), lq, lk, 0, scale, band=band,
                                       sink=None if sink is None else f32np(sink))
    kw.setdefault("input_layout", layout)
    if kv8:
        kw.update(dequant_scale_key=ks.to(DEV), dequant_scale_value=vs.to(DEV))
    if sink is not None:
        kw["learnable_sink"] = sink.to(DEV)
    if out8:
        kw["quant_scale_out"] = torch.tensor([30.0], device=DEV)
    case = dict(b=b, hq=hq, hkv=hkv, d=d, layout=layout, paged=paged, kv8=kv8, sink=sink_on, out8=out8, mode=mode,
                lq=lq, lk=lk)
    print("case", case, flush=True)
    out, lse = V2(qd, kd, vd, actual_seq_qlen=lq, actual_seq_kvlen=lk, num_query_heads=hq, num_key_value_heads=hkv,
                  softmax_scale=scale, return_softmax_lse=True, **kw, **extra)
    got = _from_layout(out.cpu(), layout, hq)
    # rows past each sequence's query length are not compared (their contents are not fixed)
    for i in range(b):
        if out8:
            w8 = G.quant_attention_out(want[i:i + 1, :lq[i]], [30.0]).astype(np.int32)
            assert np.abs(got[i, :lq[i]].numpy().astype(np.int32) - w8).max() <= 1, case
        else:
            assert_close(f32np(got[i, :lq[i]]), want[i, :lq[i]])
    lse_np = lse.cpu().numpy().reshape(b, hq, sq)
    for i in range(b):
        np.testing.assert_allclose(np.where(np.isfinite(lse_np[i, :, :lq[i]]), lse_np[i, :, :lq[i]], -1e30),
                                   np.where(np.isfinite(wl[i, :, :lq[i]]), wl[i, :, :lq[i]], -1e30),
                                   # int8 one-token decode rounds q * key scale to bf16 for the MFMA
                                   rtol=1e-3, atol=1e-2 if kv8 else 1e-3, err_msg=str(case))
