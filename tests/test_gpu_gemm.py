"""GPU parity: npu_quant_matmul and npu_grouped_matmul (W8A8, exact int32 accumulation)."""
import numpy as np
import pytest
import torch

import torchair_amd  # noqa: F401
from oracle import golden as G
from tests.helpers import assert_close, assert_int8_close, f32np, gen, rand_i8, uniform

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _exact_f64(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Exact integer product on the GPU through float64 (|sums| < 2**53): a size-independent checker."""
    return torch.matmul(a.to(torch.float64), b.to(torch.float64)).round().to(torch.int64)


@pytest.mark.parametrize("m,k,n", [(128, 2048, 11264), (128, 5632, 2048), (1, 64, 64), (300, 80, 260),
                                   (129, 1024, 384), (5, 48, 100), (17, 50, 36)])
@pytest.mark.parametrize("layout", ["kn", "nk"])
def test_quant_matmul_int32_exact(m, k, n, layout):
    g = gen(10)
    x1 = rand_i8((m, k), g)
    w = rand_i8((k, n), g)
    x2 = w if layout == "kn" else w.t().contiguous().t()  # [K,N] view of a [N,K] storage
    out = torch.ops.npu.npu_quant_matmul(x1.to(DEV), x2.to(DEV), torch.ones(1, device=DEV),
                                         output_dtype=torch.int32)
    want = G.quant_matmul(x1.numpy(), w.numpy(), out_dtype="int32")
    np.testing.assert_array_equal(out.cpu().numpy(), want)


@pytest.mark.parametrize("out_dtype,name", [(torch.bfloat16, "bf16"), (torch.float16, "fp16"), (torch.float32, "fp32")])
def test_quant_matmul_dequant_epilogue(out_dtype, name):
    g = gen(11)
    m, k, n = 128, 5632, 2048
    x1, w = rand_i8((m, k), g), rand_i8((k, n), g)
    scale, pts = uniform((n,), g, 1e-3, 1e-2), uniform((m,), g, 1e-3, 1e-2)
    out = torch.ops.npu.npu_quant_matmul(x1.to(DEV), w.to(DEV), scale.to(DEV), pertoken_scale=pts.to(DEV),
                                         output_dtype=out_dtype)
    assert out.dtype == out_dtype
    want = G.quant_matmul(x1.numpy(), w.numpy(), scale.numpy(), pts.numpy(), None, name)
    assert_close(f32np(out), want)


def test_quant_matmul_bias():
    g = gen(12)
    x1, w = rand_i8((64, 256), g), rand_i8((256, 192), g)
    bi = torch.randint(-5000, 5000, (192,), generator=g, dtype=torch.int32)
    out = torch.ops.npu.npu_quant_matmul(x1.to(DEV), w.to(DEV), torch.ones(1, device=DEV), bias=bi.to(DEV),
                                         output_dtype=torch.int32)
    np.testing.assert_array_equal(out.cpu().numpy(), G.quant_matmul(x1.numpy(), w.numpy(), bias=bi.numpy(),
                                                                     out_dtype="int32"))
    scale = uniform((192,), g, 1e-3, 1e-2)
    bf = uniform((192,), g, -1, 1)
    out = torch.ops.npu.npu_quant_matmul(x1.to(DEV), w.to(DEV), scale.to(DEV), bias=bf.to(DEV),
                                         output_dtype=torch.bfloat16)
    assert_close(f32np(out), G.quant_matmul(x1.numpy(), w.numpy(), scale.numpy(), None, bf.numpy(), "bf16"))


# Skinny path (m <= 128, k % 64 == 0, n % 16 == 0): row fragments of 1, 2 and 4 x 32 rows, 32- and
# 64-column slabs, K split over workgroups or not, slabs cut by the end of N, waves left without a stage.
@pytest.mark.parametrize("m,k,n", [(1, 2048, 11264), (31, 640, 4112), (33, 5632, 2048), (64, 64, 80),
                                   (65, 128, 176), (100, 4096, 8192), (128, 192, 16), (128, 2048, 11264),
                                   (5, 8192, 256), (64, 12288, 512)])
@pytest.mark.parametrize("layout", ["kn", "nk"])
def test_quant_matmul_skinny_exact(m, k, n, layout):
    g = gen(14)
    x1 = rand_i8((m, k), g)
    w = rand_i8((k, n), g)
    x2 = w if layout == "kn" else w.t().contiguous().t()
    out = torch.ops.npu.npu_quant_matmul(x1.to(DEV), x2.to(DEV), torch.ones(1, device=DEV),
                                         output_dtype=torch.int32)
    np.testing.assert_array_equal(out.cpu().numpy(), G.quant_matmul(x1.numpy(), w.numpy(), out_dtype="int32"))


@pytest.mark.parametrize("m,k,n", [(7, 1024, 11264), (128, 5632, 2048), (64, 12288, 512)])
@pytest.mark.parametrize("out_dtype,name", [(torch.bfloat16, "bf16"), (torch.float16, "fp16"), (torch.float32, "fp32")])
def test_quant_matmul_skinny_epilogue(m, k, n, out_dtype, name):
    g = gen(15)
    x1, w = rand_i8((m, k), g), rand_i8((k, n), g)
    scale, pts = uniform((n,), g, 1e-3, 1e-2), uniform((m,), g, 1e-3, 1e-2)
    bf = uniform((n,), g, -1, 1)
    out = torch.ops.npu.npu_quant_matmul(x1.to(DEV), w.to(DEV), scale.to(DEV), pertoken_scale=pts.to(DEV),
                                         bias=bf.to(DEV), output_dtype=out_dtype)
    assert_close(f32np(out), G.quant_matmul(x1.numpy(), w.numpy(), scale.numpy(), pts.numpy(), bf.numpy(), name))
    bi = torch.randint(-5000, 5000, (n,), generator=g, dtype=torch.int32)
    out = torch.ops.npu.npu_quant_matmul(x1.to(DEV), w.to(DEV), torch.ones(1, device=DEV), bias=bi.to(DEV),
                                         output_dtype=torch.int32)
    np.testing.assert_array_equal(out.cpu().numpy(), G.quant_matmul(x1.numpy(), w.numpy(), bias=bi.numpy(),
                                                                     out_dtype="int32"))


# Tall dense GEMMs with a [K, N] weight transpose it into the workspace first (M >= 4096, N % 256 == 0).
@pytest.mark.parametrize("m,k,n,out_dtype", [(4096, 320, 768, torch.int32), (4100, 1024, 512, torch.bfloat16),
                                             (4096, 256, 300, torch.int32)])
def test_quant_matmul_tall_kn(m, k, n, out_dtype):
    g = gen(16)
    x1, w = rand_i8((m, k), g), rand_i8((k, n), g)
    scale, pts = uniform((n,), g, 1e-3, 1e-2), uniform((m,), g, 1e-3, 1e-2)
    if out_dtype == torch.int32:
        out = torch.ops.npu.npu_quant_matmul(x1.to(DEV), w.to(DEV), torch.ones(1, device=DEV), output_dtype=torch.int32)
        np.testing.assert_array_equal(out.cpu().numpy(), G.quant_matmul(x1.numpy(), w.numpy(), out_dtype="int32"))
    else:
        out = torch.ops.npu.npu_quant_matmul(x1.to(DEV), w.to(DEV), scale.to(DEV), pertoken_scale=pts.to(DEV),
                                             output_dtype=out_dtype)
        assert_close(f32np(out), G.quant_matmul(x1.numpy(), w.numpy(), scale.numpy(), pts.numpy(), None, "bf16"))


def test_quant_matmul_large_exact_vs_f64():
    """8192^3 demonstrator shape: exact against a float64 GPU product."""
    g = torch.Generator(device=DEV)
    g.manual_seed(13)
    a = torch.randint(-127, 128, (8192, 8192), generator=g, device=DEV, dtype=torch.int8)
    b = torch.randint(-127, 128, (8192, 8192), generator=g, device=DEV, dtype=torch.int8)
    out = torch.ops.npu.npu_quant_matmul(a, b, torch.ones(1, device=DEV), output_dtype=torch.int32)
    ref = _exact_f64(a, b)
    assert torch.equal(out.to(torch.int64), ref)


def _gmm_case(g, e, m_rows, k, n, counts=None):
    if counts is None:
        counts = torch.randint(0, 2 * m_rows // e + 1, (e,), generator=g, dtype=torch.int64)
    m = int(counts.sum()) + 5
    x = rand_i8((m, k), g)
    w = rand_i8((e, k, n), g)
    return x, w, counts


@pytest.mark.parametrize("list_type", [0, 1])
@pytest.mark.parametrize("layout", ["kn", "nk"])
def test_grouped_matmul_int32_exact(list_type, layout):
    g = gen(20)
    x, w, counts = _gmm_case(g, 8, 600, 512, 256)
    counts[3] = 0  # an empty group
    gl = counts if list_type == 1 else torch.cumsum(counts, 0)
    wd = w.to(DEV) if layout == "kn" else w.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
    out = torch.ops.npu.npu_grouped_matmul([x.to(DEV)], [wd], group_list=gl.to(DEV), split_item=3, group_type=0,
                                           group_list_type=list_type, output_dtype=torch.int32)[0]
    want = G.grouped_matmul(x.numpy(), w.numpy(), gl.numpy(), list_type, out_dtype="int32")
    np.testing.assert_array_equal(out.cpu().numpy(), want)


def test_grouped_matmul_bf16_epilogue():
    g = gen(21)
    x, w, counts = _gmm_case(g, 16, 900, 256, 384)
    scale = uniform((16, 384), g, 1e-3, 1e-2)
    pts = uniform((x.shape[0],), g, 1e-3, 1e-2)
    out = torch.ops.npu.npu_grouped_matmul([x.to(DEV)], [w.to(DEV)], scale=[scale.to(DEV)],
                                           per_token_scale=[pts.to(DEV)], group_list=counts.to(DEV), split_item=3,
                                           group_type=0, group_list_type=1, output_dtype=torch.bfloat16)[0]
    want = G.grouped_matmul(x.numpy(), w.numpy(), counts.numpy(), 1, scale.numpy(), pts.numpy(), None, "bf16")
    assert_close(f32np(out), want)


def test_grouped_matmul_cfg4_gate_up_exact_vs_f64():
    """Full cfg4 gate_up shape (256 experts, 7168 -> 4096): exact against float64 per expert."""
    g = torch.Generator(device=DEV)
    g.manual_seed(22)
    e, k, n, m = 256, 7168, 4096, 32768
    counts = torch.bincount(torch.randint(0, e, (m,), generator=g, device=DEV), minlength=e).to(torch.int64)
    x = torch.randint(-127, 128, (m, k), generator=g, device=DEV, dtype=torch.int8)
    w = torch.randint(-127, 128, (e, k, n), generator=g, device=DEV, dtype=torch.int8)
    out = torch.ops.npu.npu_grouped_matmul([x], [w], group_list=counts, split_item=3, group_type=0,
                                           group_list_type=1, output_dtype=torch.int32)[0]
    ends = torch.cumsum(counts, 0).tolist()
    begin = 0
    for ei in list(range(0, e, 37)) + [e - 1]:
        b0 = 0 if ei == 0 else ends[ei - 1]
        b1 = ends[ei]
        if b1 > b0:
            ref = _exact_f64(x[b0:b1], w[ei])
            assert torch.equal(out[b0:b1].to(torch.int64), ref), f"expert {ei}"
    del begin


# int8 output (the converter's default when output_dtype is None): fp32 dequant, + offset, rint, saturate.
@pytest.mark.parametrize("m,k,n,layout", [(64, 2048, 1024, "kn"), (512, 1024, 512, "nk"), (4096, 256, 512, "kn"),
                                          (5, 48, 100, "kn")])
def test_quant_matmul_int8_output(m, k, n, layout):
    g = gen(17)
    x1, w = rand_i8((m, k), g), rand_i8((k, n), g)
    scale = uniform((n,), g, 1e-4, 4e-4)  # keeps most outputs inside int8, some saturate
    off = uniform((n,), g, -3.0, 3.0)
    bi = torch.randint(-5000, 5000, (n,), generator=g, dtype=torch.int32)
    x2 = w if layout == "kn" else w.t().contiguous().t()
    out = torch.ops.npu.npu_quant_matmul(x1.to(DEV), x2.to(DEV), scale.to(DEV), offset=off.to(DEV), bias=bi.to(DEV))
    assert out.dtype == torch.int8
    want = G.quant_matmul(x1.numpy(), w.numpy(), scale.numpy(), None, bi.numpy(), "int8", offset=off.numpy())
    assert_int8_close(out.cpu().numpy(), want)
    if k >= 256:
        assert (want == 127).any() and (want == -128).any()  # saturation is exercised


# Multi-tensor npu_grouped_matmul: one x per group (group_list absent) with per-group weights, scales and
# biases (split_item 0/1: one output per group, 2/3: concatenated), and one x with groups along M
# returned per group (split_item 0/1).
@pytest.mark.parametrize("split_item", [0, 1, 2, 3])
def test_grouped_matmul_multi_tensor(split_item):
    g = gen(23)
    ms, k, n = [37, 0, 129], 256, 192
    xs = [rand_i8((m, k), g) for m in ms]
    ws = [rand_i8((k, n), g) for _ in ms]
    scs = [uniform((n,), g, 1e-3, 1e-2) for _ in ms]
    bis = [uniform((n,), g, -1, 1) for _ in ms]
    pts = uniform((sum(ms),), g, 1e-3, 1e-2)
    outs = torch.ops.npu.npu_grouped_matmul([x.to(DEV) for x in xs], [w.to(DEV) for w in ws],
                                            scale=[s.to(DEV) for s in scs], bias=[b.to(DEV) for b in bis],
                                            per_token_scale=[pts.to(DEV)], split_item=split_item,
                                            output_dtype=torch.bfloat16)
    wants, r0 = [], 0
    for x, w, s, b, m in zip(xs, ws, scs, bis, ms):
        wants.append(G.quant_matmul(x.numpy(), w.numpy(), s.numpy(), pts[r0:r0 + m].numpy(), b.numpy(), "bf16"))
        r0 += m
    if split_item in (2, 3):
        assert len(outs) == 1
        assert_close(f32np(outs[0]), np.concatenate(wants, 0))
    else:
        assert len(outs) == 3
        for o, want in zip(outs, wants):
            assert_close(f32np(o), want)


def test_grouped_matmul_per_group_outputs():
    g = gen(24)
    x, w, counts = _gmm_case(g, 6, 400, 128, 256)
    whole = torch.ops.npu.npu_grouped_matmul([x.to(DEV)], [w.to(DEV)], group_list=counts.to(DEV), split_item=3,
                                             group_type=0, group_list_type=1, output_dtype=torch.int32)[0]
    parts = torch.ops.npu.npu_grouped_matmul([x.to(DEV)], [w.to(DEV)], group_list=counts.tolist(), split_item=0,
                                             group_type=0, group_list_type=1, output_dtype=torch.int32)
    assert [p.shape[0] for p in parts] == counts.tolist()
    torch.testing.assert_close(torch.cat(parts, 0), whole[:int(counts.sum())], rtol=0, atol=0)


@pytest.mark.parametrize("dt", [torch.int64, torch.uint64])
def test_packed_int64_scales_are_refused(dt):
    """npu_trans_quant_param packs scales into int64 words; the ops refuse them instead of converting
    the words numerically."""
    g = gen(25)
    x, w = rand_i8((8, 64), g).to(DEV), rand_i8((64, 32), g).to(DEV)
    scale = torch.ones(32, dtype=dt, device=DEV)
    with pytest.raises(RuntimeError, match="packed int64 scales"):
        torch.ops.npu.npu_quant_matmul(x, w, scale, output_dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="packed int64 scales"):
        torch.ops.npu.npu_grouped_matmul([x], [w.unsqueeze(0)], scale=[scale.unsqueeze(0)],
                                         group_list=torch.tensor([8], device=DEV), split_item=3, group_type=0,
                                         group_list_type=1, output_dtype=torch.bfloat16)


@pytest.mark.parametrize("out", ["int32", "bf16"])
def test_grouped_matmul_mixed_tiles(out):
    """[K, N] weights with n % 512 == 0 run 128 x 512 and 256 x 256 tiles side by side: groups of
    1 to 5 row slots of 128 (odd last slots stay 128 x 512), an empty group and 5 trailing rows past
    the grouped total (zero-filled)."""
    g = gen(26)
    counts = torch.tensor([1, 128, 129, 256, 0, 257, 384, 385, 600, 64], dtype=torch.int64)
    x, w, counts = _gmm_case(g, len(counts), 0, 192, 1024, counts)
    kw = {}
    if out == "bf16":
        sc = uniform((len(counts), 1024), g, 1e-3, 1e-2)
        pts = uniform((x.shape[0],), g, 1e-3, 1e-2)
        kw = dict(scale=[sc.to(DEV)], per_token_scale=[pts.to(DEV)])
    got = torch.ops.npu.npu_grouped_matmul([x.to(DEV)], [w.to(DEV)], group_list=counts.to(DEV), split_item=3,
                                           group_type=0, group_list_type=1,
                                           output_dtype=torch.int32 if out == "int32" else torch.bfloat16, **kw)[0]
    acc = G.grouped_matmul(x.numpy(), w.numpy(), counts.numpy(), 1, out_dtype="int32")
    if out == "int32":
        np.testing.assert_array_equal(got.cpu().numpy(), acc)
    else:
        want = G.grouped_matmul(x.numpy(), w.numpy(), counts.numpy(), 1, scale=sc.numpy(), per_token_scale=pts.numpy(),
                                out_dtype="bf16")
        np.testing.assert_array_equal(f32np(got), want)


def test_quant_matmul_kn_weight_prepacked_once_and_refreshed_on_write():
    """A tall product with a [K, N] weight runs the [N, K] kernel on a copy transposed once per weight:
    exact on the first call and on a repeat, and again after the weight is written in place."""
    from torchair_amd import _ops_impl
    g = gen(27)
    m, k, n = 4096, 512, 768
    x = rand_i8((m, k), g).to(DEV)
    w = rand_i8((k, n), g).to(DEV)
    for step in range(3):
        if step == 2:
            w.mul_(-1)  # in place: the cached copy is stale and must be rebuilt
        got = torch.ops.npu.npu_quant_matmul(x, w, torch.ones(1, device=DEV), output_dtype=torch.int32)
        np.testing.assert_array_equal(got.cpu().numpy(), G.int_matmul(x.cpu().numpy(), w.cpu().numpy()))
        assert id(w) in _ops_impl._NK_CACHE
