"""GPU parity: npu_add_rms_norm(_dynamic_quant), npu_scatter_pa_kv_cache and
npu_kv_rmsnorm_rope_cache against the CPU oracle."""
import numpy as np
import pytest
import torch

import torchair_amd  # noqa: F401
from oracle import golden as G
from tests.helpers import assert_close, assert_int8_close, f32np, gen, randn, uniform

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAMES = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}


# ----------------------------------------------------------------------------- add_rms_norm
@pytest.mark.parametrize("shape", [(128, 2048), (4096, 7168), (2, 3, 576), (5, 8), (3, 1000), (1, 16384)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_add_rms_norm(shape, dtype):
    g = gen(3)
    x1, x2 = randn(shape, g, dtype), randn(shape, g, dtype)
    gamma = uniform(shape[-1:], g, 0.5, 1.5).to(dtype)
    y, rstd, x = torch.ops.npu.npu_add_rms_norm(x1.to(DEV), x2.to(DEV), gamma.to(DEV), 1e-6)
    wy, wr, wx = G.add_rms_norm(f32np(x1), f32np(x2), f32np(gamma), 1e-6, NAMES[dtype])
    assert y.dtype == dtype and rstd.shape == tuple(list(shape[:-1]) + [1]) and x.shape == x1.shape
    np.testing.assert_array_equal(f32np(x), wx)  # the sum is exact before one rounding
    np.testing.assert_allclose(rstd.cpu().numpy(), wr, rtol=1e-5)
    assert_close(f32np(y), wy)


@pytest.mark.parametrize("shape", [(128, 2048), (4096, 7168), (7, 24), (3, 1000)])
def test_add_rms_norm_dynamic_quant(shape):
    g = gen(4)
    dtype = torch.bfloat16
    x1, x2 = randn(shape, g, dtype), randn(shape, g, dtype)
    gamma = uniform(shape[-1:], g, 0.5, 1.5).to(dtype)
    sm1, sm2 = uniform(shape[-1:], g, 0.5, 2.0), uniform(shape[-1:], g, 0.5, 2.0)
    beta = randn(shape[-1:], g, dtype)
    y1, y2, x, s1, s2 = torch.ops.npu.npu_add_rms_norm_dynamic_quant(
        x1.to(DEV), x2.to(DEV), gamma.to(DEV), smooth_scale1=sm1.to(DEV), smooth_scale2=sm2.to(DEV),
        beta=beta.to(DEV), epsilon=1e-6, output_mask=[True, True])
    w1, w2, wx, ws1, ws2 = G.add_rms_norm_dynamic_quant(f32np(x1), f32np(x2), f32np(gamma), f32np(sm1), f32np(sm2),
                                                        f32np(beta), 1e-6, True, "bf16")
    assert_int8_close(y1.cpu().numpy(), w1)
    assert_int8_close(y2.cpu().numpy(), w2)
    np.testing.assert_array_equal(f32np(x), wx)
    np.testing.assert_allclose(s1.cpu().numpy(), ws1, rtol=1e-5)
    np.testing.assert_allclose(s2.cpu().numpy(), ws2, rtol=1e-5)


def test_fused_equals_composed_on_gpu():
    # the rewrite of the fusion pass must not change outputs: fused vs add_rms_norm + dynamic_quant
    g = gen(5)
    x1, x2 = randn((256, 7168), g).to(DEV), randn((256, 7168), g).to(DEV)
    gamma = uniform((7168,), g, 0.5, 1.5).to(torch.bfloat16).to(DEV)
    sm = uniform((7168,), g, 0.5, 2.0).to(DEV)
    y, _, x = torch.ops.npu.npu_add_rms_norm(x1, x2, gamma)
    q, s = torch.ops.npu.npu_dynamic_quant(y, smooth_scales=sm)
    fq, _, fx, fs, _ = torch.ops.npu.npu_add_rms_norm_dynamic_quant(x1, x2, gamma, smooth_scale1=sm,
                                                                    output_mask=[True, False])
    assert torch.equal(q, fq) and torch.equal(s, fs) and torch.equal(x, fx)


# ----------------------------------------------------------------------------- scatter_pa_kv_cache
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.int8, torch.float32])
@pytest.mark.parametrize("slot_dtype", [torch.int32, torch.int64])
def test_scatter_pa_kv_cache_norm(dtype, slot_dtype):
    g = gen(6)
    t, h, dk, dv, nb, bs = 37, 8, 128, 64, 10, 16
    if dtype == torch.int8:
        key = torch.randint(-127, 128, (t, h, dk), generator=g, dtype=torch.int8)
        val = torch.randint(-127, 128, (t, h, dv), generator=g, dtype=torch.int8)
    else:
        key, val = randn((t, h, dk), g, dtype), randn((t, h, dv), g, dtype)
    kc = torch.zeros(nb, bs, h, dk, dtype=dtype)
    vc = torch.zeros(nb, bs, h, dv, dtype=dtype)
    slots = torch.randperm(nb * bs, generator=g)[:t].to(slot_dtype)
    slots[3] = -1
    kd, vd = kc.to(DEV), vc.to(DEV)
    torch.ops.npu.npu_scatter_pa_kv_cache(key.to(DEV), val.to(DEV), kd, vd, slots.to(DEV))
    to_np = (lambda a: a.numpy()) if dtype in (torch.int8, torch.float32) else f32np
    wk, wv = G.scatter_pa_kv_cache(to_np(key), to_np(val), to_np(kc), to_np(vc), slots.numpy(), "Norm")
    np.testing.assert_array_equal(to_np(kd.cpu()), wk)
    np.testing.assert_array_equal(to_np(vd.cpu()), wv)


def test_scatter_pa_kv_cache_nz_reference_smoke_shapes():
    # tests/smoke/ge_test.py:244-267 (fp16, PA_NZ caches), through the functional op
    g = gen(7)
    t, h, dk, dv, nb, bs, last = 16, 4, 32, 64, 2, 32, 16
    key, val = randn((t, h, dk), g, torch.float16), randn((t, h, dv), g, torch.float16)
    kc = randn((nb, h * dk // last, bs, last), g, torch.float16)
    vc = torch.zeros(nb, h * dv // last, bs, last, dtype=torch.float16)
    slots = torch.randperm(nb * bs, generator=g)[:t].to(torch.int32)
    ko, vo = torch.ops.npu.npu_scatter_pa_kv_cache_functional(key.to(DEV), val.to(DEV), kc.to(DEV), vc.to(DEV),
                                                              slots.to(DEV), cache_mode="PA_NZ")
    wk, wv = G.scatter_pa_kv_cache(f32np(key), f32np(val), f32np(kc), f32np(vc), slots.numpy(), "PA_NZ")
    np.testing.assert_array_equal(f32np(ko), wk)
    np.testing.assert_array_equal(f32np(vo), wv)


# ----------------------------------------------------------------------------- kv_rmsnorm_rope_cache
def _mla(g, b, s, dc=512, dr=64, dtype=torch.bfloat16):
    kv = randn((b, 1, s, dc + dr), g, dtype)
    gamma = uniform((dc,), g, 0.5, 1.5).to(dtype)
    theta = uniform((b, 1, s, dr // 2), g, -3.0, 3.0)
    cos = torch.cat([theta.cos()] * 2, -1).to(dtype)
    sin = torch.cat([theta.sin()] * 2, -1).to(dtype)
    return kv, gamma, cos, sin


def test_kv_rmsnorm_rope_cache_pa_bf16():
    g = gen(8)
    b, s, nb, bs = 4, 3, 6, 16
    kv, gamma, cos, sin = _mla(g, b, s)
    idx = torch.randperm(nb * bs, generator=g)[:b * s].to(torch.int64)
    idx[2] = -1
    kc = torch.zeros(nb, bs, 1, 64, dtype=torch.bfloat16)
    cc = torch.zeros(nb, bs, 1, 512, dtype=torch.bfloat16)
    kd, cd = kc.to(DEV), cc.to(DEV)
    kr, ckv = torch.ops.npu.npu_kv_rmsnorm_rope_cache_v2(kv.to(DEV), gamma.to(DEV), cos.to(DEV), sin.to(DEV),
                                                         idx.to(DEV), kd, cd, epsilon=1e-5, cache_mode="PA")
    wk, wc, wkr, wckv = G.kv_rmsnorm_rope_cache(f32np(kv), f32np(gamma), f32np(cos), f32np(sin), idx.numpy(),
                                                f32np(kc), f32np(cc), 1e-5, "PA")
    np.testing.assert_array_equal(f32np(kr), wkr)  # RoPE is exact: fp32 products and sums, one rounding
    assert_close(f32np(ckv), wckv)
    np.testing.assert_array_equal(f32np(kd.cpu()), wk)
    assert_close(f32np(cd.cpu()), wc)


def test_kv_rmsnorm_rope_cache_norm_layout_functional():
    g = gen(9)
    b, s, scache = 2, 5, 8
    kv, gamma, cos, sin = _mla(g, b, s)
    pos = torch.tensor([[0, 2, 4, 6, 7], [1, 3, -1, 5, 0]], dtype=torch.int64)
    kc = randn((b, 1, scache, 64), g)
    cc = randn((b, 1, scache, 512), g)
    kr, ckv, ko, co = torch.ops.npu.npu_kv_rmsnorm_rope_cache_v2_functional(
        kv.to(DEV), gamma.to(DEV), cos.to(DEV), sin.to(DEV), pos.to(DEV), kc.to(DEV), cc.to(DEV), cache_mode="Norm")
    wk, wc, wkr, wckv = G.kv_rmsnorm_rope_cache(f32np(kv), f32np(gamma), f32np(cos), f32np(sin), pos.numpy(),
                                                f32np(kc), f32np(cc), 1e-5, "Norm")
    np.testing.assert_array_equal(f32np(ko), wk)
    assert_close(f32np(co), wc)
    assert_close(f32np(ckv), wckv)


def test_kv_rmsnorm_rope_cache_int8_per_token_feeds_mla_decode():
    # the writer produces the int8 latent + per-token scale cache the MLA decode kernel reads
    g = gen(10)
    b, s, nb, bs = 2, 64, 4, 32
    kv, gamma, cos, sin = _mla(g, b, s)
    slots = torch.arange(b * s, dtype=torch.int64)  # batch 0 -> blocks 0, 1; batch 1 -> blocks 2, 3
    kc = torch.zeros(nb, bs, 1, 64, dtype=torch.bfloat16, device=DEV)
    cc = torch.zeros(nb, bs, 1, 512, dtype=torch.int8, device=DEV)
    tok = torch.zeros(nb, bs, dtype=torch.float32, device=DEV)
    _, ckv = torch.ops.npu.npu_kv_rmsnorm_rope_cache_v2(kv.to(DEV), gamma.to(DEV), cos.to(DEV), sin.to(DEV),
                                                        slots.to(DEV), kc, cc, c_kv_scale=tok, cache_mode="PA")
    _, wc, _, wckv, wts = G.kv_rmsnorm_rope_cache(f32np(kv), f32np(gamma), f32np(cos), f32np(sin), slots.numpy(),
                                                  np.zeros((nb, bs, 1, 64), np.float32),
                                                  np.zeros((nb, bs, 1, 512), np.int8), 1e-5, "PA",
                                                  c_kv_token_scale=np.zeros((nb, bs), np.float32))
    assert_int8_close(cc.cpu().numpy(), wc)
    np.testing.assert_allclose(tok.cpu().numpy(), wts, rtol=1e-5)
    # decode over the written cache equals attention over the dequantised latent
    hq = 16
    qn, qr = randn((b, 1, hq, 512), g), randn((b, 1, hq, 64), g)
    bt = torch.tensor([[0, 1], [2, 3]], dtype=torch.int32)
    lens = [s, s]
    out, _ = torch.ops.air.npu_fused_infer_attention_score(
        qn.to(DEV), cc, cc, query_rope=qr.to(DEV), key_rope=kc, key_antiquant_scale=tok, key_antiquant_mode=1,
        block_table=bt.to(DEV), actual_seq_lengths_kv=torch.tensor(lens, device=DEV), num_heads=hq,
        num_key_value_heads=1, input_layout="BSND", block_size=bs, scale=1.0 / 192 ** 0.5)
    want, _ = G.mla_decode_attention(f32np(qn)[:, 0], f32np(qr)[:, 0], cc[:, :, 0].cpu().numpy(), tok.cpu().numpy(),
                                     f32np(kc[:, :, 0].cpu()), bt.numpy(), lens, 1.0 / 192 ** 0.5)
    assert_close(f32np(out[:, 0].cpu()), want)


@pytest.mark.parametrize("seed", range(8))
def test_add_rms_norm_family_random(seed):
    """Seeded random shapes (leading dims 1-3, widths on and off the vector paths, few and many rows),
    dtypes, the optional smooth scales and beta, and one or two quantised outputs, against the oracle."""
    rng = np.random.default_rng(9000 + seed)
    g = gen(9000 + seed)
    h = int(rng.choice([8, 24, 1000, 2048, 5120, 7168, 7170]))
    lead = [int(x) for x in rng.integers(1, 12, int(rng.integers(1, 4)))]
    if rng.random() < 0.3:
        lead = [int(rng.integers(500, 3000))]  # many rows (the total stays at most a few thousand)
    shape = tuple(lead) + (h,)
    dtype = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(0, 3))]
    x1, x2 = randn(shape, g, dtype), randn(shape, g, dtype)
    gamma = uniform((h,), g, 0.5, 1.5).to(dtype)
    print("case", dict(shape=shape, dtype=str(dtype)), flush=True)
    y, rstd, x = torch.ops.npu.npu_add_rms_norm(x1.to(DEV), x2.to(DEV), gamma.to(DEV), 1e-6)
    wy, wr, wx = G.add_rms_norm(f32np(x1), f32np(x2), f32np(gamma), 1e-6, NAMES[dtype])
    np.testing.assert_array_equal(f32np(x), wx)
    np.testing.assert_allclose(rstd.cpu().numpy().reshape(wr.shape), wr, rtol=1e-5)
    assert_close(f32np(y), wy)
    if dtype == torch.float32:
        return  # the fused quantising op takes half-precision inputs
    sm1 = uniform((h,), g, 0.5, 2.0) if rng.random() < 0.7 else None
    second = sm1 is not None and rng.random() < 0.5
    sm2 = uniform((h,), g, 0.5, 2.0) if second else None
    beta = randn((h,), g, dtype) if rng.random() < 0.5 else None
    dv = lambda v: None if v is None else v.to(DEV)  # noqa: E731
    y1, y2, xo, s1, s2 = torch.ops.npu.npu_add_rms_norm_dynamic_quant(
        x1.to(DEV), x2.to(DEV), gamma.to(DEV), smooth_scale1=dv(sm1), smooth_scale2=dv(sm2), beta=dv(beta),
        epsilon=1e-6, output_mask=[True, second])
    npf = lambda v: None if v is None else f32np(v)  # noqa: E731
    w1, w2, wx2, ws1, ws2 = G.add_rms_norm_dynamic_quant(f32np(x1), f32np(x2), f32np(gamma), npf(sm1), npf(sm2),
                                                         npf(beta), 1e-6, second, NAMES[dtype])
    assert_int8_close(y1.cpu().numpy(), w1)
    np.testing.assert_array_equal(f32np(xo), wx2)
    np.testing.assert_allclose(s1.cpu().numpy().reshape(ws1.shape), ws1, rtol=1e-5)
    if second:
        assert_int8_close(y2.cpu().numpy(), w2)
        np.testing.assert_allclose(s2.cpu().numpy().reshape(ws2.shape), ws2, rtol=1e-5)


@pytest.mark.parametrize("seed", range(8))
def test_scatter_pa_kv_cache_random(seed):
    """Seeded random npu_scatter_pa_kv_cache: token counts, heads, key / value widths, block counts and
    sizes, dtypes, both cache layouts, skipped (negative) slots, int32 / int64 slot mappings."""
    rng = np.random.default_rng(9500 + seed)
    g = gen(9500 + seed)
    dtype = [torch.bfloat16, torch.float16, torch.int8, torch.float32][int(rng.integers(0, 4))]
    mode = "PA_NZ" if rng.random() < 0.4 else "Norm"
    esz = torch.tensor([], dtype=dtype).element_size()
    last = 32 // esz
    h = int(rng.integers(1, 9))
    dk = last * int(rng.integers(1, 9))
    dv = last * int(rng.integers(1, 9))
    nb, bs = int(rng.integers(1, 12)), int(rng.choice([16, 32, 64, 128]))
    t = int(rng.integers(1, nb * bs + 1))
    if dtype == torch.int8:
        key = torch.randint(-127, 128, (t, h, dk), generator=g, dtype=torch.int8)
        val = torch.randint(-127, 128, (t, h, dv), generator=g, dtype=torch.int8)
    else:
        key, val = randn((t, h, dk), g, dtype), randn((t, h, dv), g, dtype)
    if mode == "Norm":
        kc, vc = torch.zeros(nb, bs, h, dk, dtype=dtype), torch.zeros(nb, bs, h, dv, dtype=dtype)
    else:
        kc = torch.zeros(nb, h * dk // last, bs, last, dtype=dtype)
        vc = torch.zeros(nb, h * dv // last, bs, last, dtype=dtype)
    slots = torch.randperm(nb * bs, generator=g)[:t]
    slots[torch.rand(t, generator=g) < 0.1] = -1
    slots = slots.to(torch.int32 if rng.random() < 0.5 else torch.int64)
    print("case", dict(dtype=str(dtype), mode=mode, t=t, h=h, dk=dk, dv=dv, nb=nb, bs=bs), flush=True)
    ko, vo = torch.ops.npu.npu_scatter_pa_kv_cache_functional(key.to(DEV), val.to(DEV), kc.to(DEV), vc.to(DEV),
                                                              slots.to(DEV), cache_mode=mode)
    to_np = (lambda a: a.numpy()) if dtype in (torch.int8, torch.float32) else f32np
    wk, wv = G.scatter_pa_kv_cache(to_np(key), to_np(val), to_np(kc), to_np(vc), slots.numpy(), mode)
    np.testing.assert_array_equal(to_np(ko.cpu()), wk)
    np.testing.assert_array_equal(to_np(vo.cpu()), wv)


@pytest.mark.parametrize("seed", range(6))
def test_kv_rmsnorm_rope_cache_random(seed):
    """Seeded random MLA cache writes: batch and step counts, PA (block counts and sizes) or Norm
    layouts, skipped rows, bf16 / fp16, and the int8 latent with per-token scales."""
    rng = np.random.default_rng(9700 + seed)
    g = gen(9700 + seed)
    b, s = int(rng.integers(1, 6)), int(rng.integers(1, 40))
    dtype = torch.bfloat16 if rng.random() < 0.6 else torch.float16
    kv, gamma, cos, sin = _mla(g, b, s, dtype=dtype)
    mode = "PA" if rng.random() < 0.7 else "Norm"
    int8_lat = mode == "PA" and rng.random() < 0.5
    case = dict(b=b, s=s, dtype=str(dtype), mode=mode, int8=int8_lat)
    if mode == "PA":
        bs = int(rng.choice([16, 32, 64, 128]))
        nb = (b * s + bs - 1) // bs + int(rng.integers(0, 3))
        idx = torch.randperm(nb * bs, generator=g)[:b * s].to(torch.int64)
        kc = torch.zeros(nb, bs, 1, 64, dtype=dtype)
        cc = torch.zeros(nb, bs, 1, 512, dtype=torch.int8 if int8_lat else dtype)
    else:
        scache = s + int(rng.integers(0, 8))
        idx = torch.stack([torch.randperm(scache, generator=g)[:s] for _ in range(b)]).to(torch.int64)
        kc = randn((b, 1, scache, 64), g, dtype)
        cc = randn((b, 1, scache, 512), g, dtype)
    idx.view(-1)[torch.rand(idx.numel(), generator=g) < 0.1] = -1
    case["idx"] = tuple(idx.shape)
    print("case", case, flush=True)
    kd, cd = kc.to(DEV), cc.to(DEV)
    kw = {}
    tok = None
    if int8_lat:
        tok = torch.zeros(kc.shape[0], kc.shape[1], dtype=torch.float32, device=DEV)
        kw["c_kv_scale"] = tok
    kr, ckv = torch.ops.npu.npu_kv_rmsnorm_rope_cache_v2(kv.to(DEV), gamma.to(DEV), cos.to(DEV), sin.to(DEV),
                                                         idx.to(DEV), kd, cd, epsilon=1e-5, cache_mode=mode, **kw)
    name = NAMES[dtype]
    res = G.kv_rmsnorm_rope_cache(f32np(kv), f32np(gamma), f32np(cos), f32np(sin), idx.numpy(), f32np(kc),
                                  cc.numpy() if int8_lat else f32np(cc), 1e-5, mode,
                                  c_kv_token_scale=np.zeros(tuple(kc.shape[:2]), np.float32) if int8_lat else None,
                                  dtype=name)
    wk, wc, wkr, wckv = res[:4]
    np.testing.assert_array_equal(f32np(kr), wkr)
    assert_close(f32np(ckv), wckv)
    np.testing.assert_array_equal(f32np(kd.cpu()), wk)
    if int8_lat:
        assert_int8_close(cd.cpu().numpy(), wc)
        np.testing.assert_allclose(tok.cpu().numpy(), res[4], rtol=1e-5)
    else:
        assert_close(f32np(cd.cpu()), wc)
