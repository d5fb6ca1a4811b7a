"""Writes the golden fixtures of tests/golden/*.npz from the CPU oracle (oracle/golden.py).

The reference holds no golden vectors for these ops (its kernels are closed CANN binaries), so the
semantics the oracle fixes (rounding, tie order, routing index conventions, padded rows) are frozen
here: tests/test_golden_fixtures.py checks that the oracle still reproduces every file bit for bit,
and that the GPU kernels match them to the parity bar. Inputs come from one seeded
torch.Generator per case. Floating inputs are stored as they are fed to the op (bf16 as uint16
bit patterns). Run: python tests/golden/make_fixtures.py
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import golden as G  # noqa: E402


def _g(seed):
    return torch.Generator().manual_seed(seed)


def _bf16(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> uint16 bit patterns."""
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _f(bits: np.ndarray) -> np.ndarray:
    return G.bf16_bits_to_f32(bits)


def case_dynamic_quant():
    g = _g(1)
    x = torch.randn(16, 256, generator=g) * 3
    x[3] = 0.0            # all-zero row: scale 0, y 0
    x[5] = -1.25          # constant row: y = -127
    x[7, 10] = 1e4        # one dominant element
    xb = _bf16(x)
    sm = (torch.rand(256, generator=g) + 0.5).numpy().astype(np.float32)
    y, s = G.dynamic_quant(_f(xb))
    ys, ss = G.dynamic_quant(_f(xb), sm)
    return dict(x=xb, smooth=sm, y=y, scale=s, y_smooth=ys, scale_smooth=ss)


def case_dequant_swiglu_quant():
    g = _g(2)
    x = torch.randint(-2 ** 20, 2 ** 20, (12, 128), generator=g, dtype=torch.int32).numpy()
    ws = (torch.rand(128, generator=g) * 9e-3 + 1e-3).numpy()
    acts = (torch.rand(12, generator=g) * 9e-3 + 1e-3).numpy()
    yl, sl = G.dequant_swiglu_quant(x, ws, acts, activate_left=True)
    yr, sr = G.dequant_swiglu_quant(x, ws, acts, activate_left=False)
    return dict(x=x, weight_scale=ws, activation_scale=acts, y_left=yl, scale_left=sl, y_right=yr, scale_right=sr)


def case_quant_matmul():
    g = _g(3)
    x1 = torch.randint(-127, 128, (24, 160), generator=g, dtype=torch.int8).numpy()
    x2 = torch.randint(-127, 128, (160, 72), generator=g, dtype=torch.int8).numpy()
    sc = (torch.rand(72, generator=g) * 9e-3 + 1e-3).numpy()
    pts = (torch.rand(24, generator=g) * 9e-3 + 1e-3).numpy()
    acc = G.quant_matmul(x1, x2, out_dtype="int32")
    bf = G.quant_matmul(x1, x2, sc, pts, None, "bf16")
    return dict(x1=x1, x2=x2, scale=sc, pertoken_scale=pts, acc=acc, out_bf16=bf)


def case_grouped_matmul():
    g = _g(4)
    counts = np.array([10, 0, 21, 7, 1], np.int64)
    x = torch.randint(-127, 128, (int(counts.sum()) + 3, 96), generator=g, dtype=torch.int8).numpy()
    w = torch.randint(-127, 128, (5, 96, 48), generator=g, dtype=torch.int8).numpy()
    sc = (torch.rand(5, 48, generator=g) * 9e-3 + 1e-3).numpy()
    pts = (torch.rand(x.shape[0], generator=g) * 9e-3 + 1e-3).numpy()
    acc = G.grouped_matmul(x, w, counts, 1, out_dtype="int32")
    bf = G.grouped_matmul(x, w, counts, 1, sc, pts, None, "bf16")
    return dict(x=x, w=w, counts=counts, scale=sc, per_token_scale=pts, acc=acc, out_bf16=bf)


def case_moe_layer():
    """gating_top_k (DeepSeek-V3 settings) -> init_routing_v2 -> finalize_routing on 16 tokens."""
    g = _g(5)
    t, e, k, h = 16, 64, 8, 32
    logits = torch.randn(t, e, generator=g).numpy()
    logits[2, 5] = logits[2, 6]  # a tie: the lower expert id wins
    bias = (torch.randn(e, generator=g) * 0.1).numpy()
    x = _bf16(torch.randn(t, h, generator=g))
    y, idx, _ = G.moe_gating_top_k(logits, k, bias, 4, 8, 1, 0, 1, False, 1.0, 1e-20)
    ex, ri, counts, _ = G.moe_init_routing_v2(_f(x), idx, None, t * k, 0, e, 1, 0)
    out = G.moe_finalize_routing(ex, None, None, None, y, ri, idx, 2, "bf16")
    return dict(logits=logits, bias=bias, x=x, weights=y, expert_idx=idx, expanded_x=G.f32_to_bf16_bits(ex),
                expanded_row_idx=ri, counts=counts, finalized=G.f32_to_bf16_bits(out))


def case_paged_decode():
    g = _g(6)
    lens = np.array([37, 0, 130, 64], np.int64)
    hq, hkv, d, bs = 8, 2, 64, 32
    nb = [(int(L) + bs - 1) // bs for L in lens]
    total = sum(nb) + 2
    perm = torch.randperm(total, generator=g).numpy()
    bt = np.zeros((len(lens), max(nb)), np.int32)
    off = 0
    for i, n in enumerate(nb):
        bt[i, :n] = perm[off:off + n]
        off += n
    kc = _bf16(torch.randn(total, bs, hkv, d, generator=g))
    vc = _bf16(torch.randn(total, bs, hkv, d, generator=g))
    q = _bf16(torch.randn(len(lens), hq, d, generator=g))
    out, lse = G.paged_decode_attention(_f(q), _f(kc), _f(vc), bt, lens, 1.0 / math.sqrt(d))
    return dict(q=q, k_cache=kc, v_cache=vc, block_table=bt, lens=lens, out=out, lse=lse)


def case_prefill():
    g = _g(7)
    b, s, hq, hkv, d = 2, 40, 4, 2, 64
    q = _bf16(torch.randn(b, s, hq, d, generator=g))
    k = _bf16(torch.randn(b, s, hkv, d, generator=g))
    v = _bf16(torch.randn(b, s, hkv, d, generator=g))
    lq = np.array([40, 17], np.int64)
    lkv = np.array([40, 29], np.int64)
    out, lse = G.prefill_attention(_f(q), _f(k), _f(v), lq, lkv, 1, 1.0 / math.sqrt(d))
    return dict(q=q, k=k, v=v, lq=lq, lkv=lkv, out=out, lse=lse)


def case_add_rms_norm_dynamic_quant():
    g = _g(8)
    x1 = _bf16(torch.randn(6, 256, generator=g))
    x2 = _bf16(torch.randn(6, 256, generator=g))
    gamma = _bf16(torch.rand(256, generator=g) + 0.5)
    sm = (torch.rand(256, generator=g) + 0.5).numpy()
    y, rstd, xo = G.add_rms_norm(_f(x1), _f(x2), _f(gamma), 1e-6, "bf16")
    res = G.add_rms_norm_dynamic_quant(_f(x1), _f(x2), _f(gamma), sm, None, None, 1e-6, "bf16")
    return dict(x1=x1, x2=x2, gamma=gamma, smooth=sm, y=G.f32_to_bf16_bits(y), rstd=rstd,
                x_out=G.f32_to_bf16_bits(xo), q_y=res[0], q_scale=res[3])


CASES = {
    "dynamic_quant": case_dynamic_quant,
    "dequant_swiglu_quant": case_dequant_swiglu_quant,
    "quant_matmul": case_quant_matmul,
    "grouped_matmul": case_grouped_matmul,
    "moe_layer": case_moe_layer,
    "paged_decode": case_paged_decode,
    "prefill": case_prefill,
    "add_rms_norm_dynamic_quant": case_add_rms_norm_dynamic_quant,
}


def main():
    for name, fn in CASES.items():
        arrays = {k: np.asarray(v) for k, v in fn().items()}
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays)
        print(name, sum(a.nbytes for a in arrays.values()), "bytes")


if __name__ == "__main__":
    main()
