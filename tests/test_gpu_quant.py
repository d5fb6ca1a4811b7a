"""GPU parity: npu_dynamic_quant and npu_dequant_swiglu_quant against the CPU oracle."""
import numpy as np
import pytest
import torch

import torchair_amd  # noqa: F401
from oracle import golden as G
from tests.helpers import assert_close, assert_int8_close, f32np, gen, randn, uniform

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _dq_check(x, smooth=None, gidx=None):
    y, s = torch.ops.npu.npu_dynamic_quant(x.to(DEV), smooth_scales=None if smooth is None else smooth.to(DEV),
                                           group_index=None if gidx is None else gidx.to(DEV))
    wy, ws = G.dynamic_quant(f32np(x), None if smooth is None else f32np(smooth),
                             None if gidx is None else gidx.numpy())
    assert y.dtype == torch.int8 and y.shape == x.shape and s.shape == x.shape[:-1]
    assert_int8_close(y.cpu().numpy(), wy)
    np.testing.assert_allclose(s.cpu().numpy(), ws, rtol=1e-6, atol=0)


@pytest.mark.parametrize("shape", [(128, 2048), (8192, 7168), (64, 16384), (3, 5, 1000), (1, 20000), (7, 8)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_dynamic_quant_shapes(shape, dtype):
    g = gen(1)
    _dq_check(randn(shape, g, dtype))


def test_dynamic_quant_smooth_and_groups():
    g = gen(2)
    x = randn((300, 512), g)
    _dq_check(x, smooth=uniform((512,), g, 0.5, 2.0))
    gidx = torch.tensor([50, 50, 200, 300], dtype=torch.int32)
    _dq_check(x, smooth=uniform((4, 512), g, 0.5, 2.0), gidx=gidx)
    _dq_check(x, smooth=uniform((4, 512), g, 0.5, 2.0), gidx=gidx.to(torch.int64))


def test_dynamic_quant_zero_and_constant_rows():
    x = torch.zeros(4, 256, dtype=torch.bfloat16)
    x[1] = 3.0
    x[2] = -0.25
    y, s = torch.ops.npu.npu_dynamic_quant(x.to(DEV))
    y, s = y.cpu(), s.cpu()
    assert s[0] == 0 and (y[0] == 0).all()
    assert (y[1] == 127).all() and (y[2] == -127).all()
    assert torch.ops.npu.npu_dynamic_quant(torch.empty(0, 64, dtype=torch.bfloat16, device=DEV))[0].numel() == 0


def _dsq_inputs(rows, n, g, groups=None):
    x = torch.randint(-200000, 200000, (rows, 2 * n), generator=g, dtype=torch.int32)
    ws_shape = (2 * n,) if groups is None else (groups, 2 * n)
    ws = uniform(ws_shape, g, 1e-3, 1e-2)
    act = uniform((rows,), g, 0.005, 0.05)
    return x, ws, act


def _dsq_check(x, ws, act, left, bias=None, qs=None, gidx=None):
    y, s = torch.ops.npu.npu_dequant_swiglu_quant(
        x.to(DEV), weight_scale=ws.to(DEV), activation_scale=None if act is None else act.to(DEV),
        bias=None if bias is None else bias.to(DEV), quant_scale=None if qs is None else qs.to(DEV),
        group_index=None if gidx is None else gidx.to(DEV), activate_left=left, quant_mode=1)
    wy, wsc = G.dequant_swiglu_quant(x.numpy(), ws.numpy(), None if act is None else act.numpy(),
                                     None if bias is None else bias.numpy(), None if qs is None else qs.numpy(),
                                     None if gidx is None else gidx.numpy(), left)
    assert y.shape == (x.shape[0], x.shape[1] // 2)
    assert_int8_close(y.cpu().numpy(), wy)
    np.testing.assert_allclose(s.cpu().numpy(), wsc, rtol=1e-5, atol=1e-30)


@pytest.mark.parametrize("left", [True, False])
def test_dsq_cfg1(left):
    g = gen(3)
    x, ws, act = _dsq_inputs(128, 5632, g)
    _dsq_check(x, ws, act, left)


def test_dsq_grouped_cfg4_slice():
    g = gen(4)
    counts = torch.randint(0, 40, (64,), generator=g, dtype=torch.int64)
    rows = int(counts.sum()) + 17  # rows past the grouped total come out as zero
    x, ws, act = _dsq_inputs(rows, 2048, g, groups=64)
    _dsq_check(x, ws, act, True, gidx=counts)


def test_dsq_many_rows_ragged_groups():
    """Config-4-sized row counts: ragged groups, empty groups, rows past the grouped total."""
    g = gen(14)
    counts = torch.randint(0, 130, (64,), generator=g, dtype=torch.int64)
    counts[5] = 0
    counts[6] = 1
    rows = int(counts.sum()) + 7
    rows += 1 if rows % 4 == 0 else 0
    assert rows >= 4096
    x, ws, act = _dsq_inputs(rows, 2048, g, groups=64)
    _dsq_check(x, ws, act, True, gidx=counts)
    x2, ws2, act2 = _dsq_inputs(4099, 2048, g)
    _dsq_check(x2, ws2, act2, False)


def test_dsq_bias_quant_scale_and_odd_n():
    g = gen(5)
    x, ws, act = _dsq_inputs(33, 100, g)
    _dsq_check(x, ws, act, False, bias=torch.randint(-1000, 1000, (200,), generator=g, dtype=torch.int32))
    _dsq_check(x, ws, None, True, bias=uniform((200,), g, -1, 1), qs=uniform((100,), g, 0.5, 2))
    x2, ws2, act2 = _dsq_inputs(9, 7, g)  # n not a multiple of 4 -> generic kernel
    _dsq_check(x2, ws2, act2, True)


# DynamicQuantV2: symmetric per tensor or with a custom range, and the asymmetric op; smooth scales with
# group_index; a zero row and an all-positive row.
@pytest.mark.parametrize("asym,quant_mode,qmax", [(False, "pertensor", 0.0), (False, "pertoken", 63.0),
                                                  (False, "pertensor", 100.0), (True, "pertoken", 0.0),
                                                  (True, "pertensor", 0.0)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_dynamic_quant_v2(asym, quant_mode, qmax, dtype):
    g = gen(5)
    x = randn((300, 1000), g, dtype)
    x[7] = 0
    x[9] = x[9].abs() + 0.25
    sm = uniform((3, 1000), g, 0.5, 2.0)
    gidx = torch.tensor([100, 250, 300], dtype=torch.int64)
    kw = dict(smooth_scales=sm.to(DEV), group_index=gidx.to(DEV), quant_mode=quant_mode, dst_type_max=qmax)
    if asym:
        y, s, off = torch.ops.npu.npu_dynamic_quant_asymmetric(x.to(DEV), **kw)
    else:
        y, s = torch.ops.npu.npu_dynamic_quant(x.to(DEV), **kw)
    wy, ws, woff = G.dynamic_quant_v2(f32np(x), f32np(sm), gidx.numpy(), symmetric=not asym,
                                      per_tensor=quant_mode == "pertensor", dst_type_max=qmax)
    assert tuple(s.shape) == ws.shape
    assert_int8_close(y.cpu().numpy(), wy)
    np.testing.assert_allclose(s.cpu().numpy(), ws, rtol=1e-6, atol=0)
    if asym:
        np.testing.assert_allclose(off.cpu().numpy(), woff, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("grouped", [False, True])
def test_dequant_swiglu_quant_static_mode(grouped):
    """quant_mode 0 (static): clamp(rint(h * quant_scale + quant_offset)), scale 0, against the oracle
    (int8 within 1 LSB on at most 0.1%: h differs from the oracle's by the SwiGLU's reciprocal)."""
    g = torch.Generator().manual_seed(90)
    rows, n = 300, 1024
    x = torch.randint(-30000, 30000, (rows, 2 * n), generator=g, dtype=torch.int32)
    ng = 4 if grouped else 1
    counts = torch.tensor([100, 0, 120, 50], dtype=torch.int64) if grouped else None
    ws = torch.rand(ng, 2 * n, generator=g) * 1e-3
    act = torch.rand(rows, generator=g) * 0.1
    qs = torch.rand(ng, n, generator=g) * 20 + 1
    qo = torch.rand(ng, n, generator=g) * 2 - 1
    y, s = torch.ops.npu.npu_dequant_swiglu_quant(
        x.to(DEV), weight_scale=ws.to(DEV), activation_scale=act.to(DEV), quant_scale=qs.to(DEV),
        quant_offset=qo.to(DEV), group_index=counts.to(DEV) if grouped else None, activate_left=True, quant_mode=0)
    wy, wsc = G.dequant_swiglu_quant(x.numpy(), ws.numpy(), act.numpy(), None, qs.numpy(),
                                     counts.numpy() if grouped else None, True, 0, qo.numpy())
    assert_int8_close(y.cpu().numpy(), wy)
    np.testing.assert_array_equal(s.cpu().numpy(), wsc)


@pytest.mark.parametrize("dt,name", [(torch.float32, "fp32"), (torch.bfloat16, "bf16"), (torch.float16, "fp16")])
@pytest.mark.parametrize("shape,dim", [((128, 11264), -1), ((6, 10, 4), 1), ((8, 3, 5), 0)])
def test_swiglu(dt, name, shape, dim):
    """npu_swiglu against the oracle: fp32 within a few ulp (the hardware exp2 and reciprocal), bf16 / fp16
    within one rounding of the output."""
    g = gen(34)
    x = (torch.randn(shape, generator=g) * 3).to(dt)
    y = torch.ops.npu.npu_swiglu(x.to(DEV), dim=dim)
    want = G.swiglu(f32np(x), dim, name)
    got = f32np(y)
    assert y.dtype == dt and got.shape == want.shape
    if dt == torch.float32:
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
    else:
        assert_close(got, want)


@pytest.mark.parametrize("left,quant_mode,grouped", [(True, 1, False), (False, 1, True), (True, 0, True)])
def test_dequant_swiglu_quant_clamped_mode(left, quant_mode, grouped):
    """swiglu_mode 1 (odd-even blocked columns, the clamped SwiGLU) against the oracle, with values on
    both sides of the clamp limit, non-default glu_alpha / glu_bias / clamp_limit, bias and groups."""
    g = torch.Generator().manual_seed(91)
    rows, n = 260, 768
    x = torch.randint(-40000, 40000, (rows, 2 * n), generator=g, dtype=torch.int32)
    ng = 3 if grouped else 1
    counts = torch.tensor([100, 0, 150], dtype=torch.int64) if grouped else None
    ws = torch.rand(ng, 2 * n, generator=g) * 4e-4  # |dequantised| up to ~16: both sides of the limit
    act = torch.rand(rows, generator=g) + 0.5
    bias = torch.randint(-500, 500, (ng, 2 * n), generator=g, dtype=torch.int32)
    qs = torch.rand(ng, n, generator=g) * 2 + 0.5
    kw = dict(weight_scale=ws.to(DEV), activation_scale=act.to(DEV), bias=bias.to(DEV), quant_scale=qs.to(DEV),
              group_index=counts.to(DEV) if grouped else None, activate_left=left, quant_mode=quant_mode,
              swiglu_mode=1, clamp_limit=6.0, glu_alpha=1.5, glu_bias=0.75)
    qo = None
    if quant_mode == 0:
        qo = torch.rand(ng, n, generator=g) * 2 - 1
        kw["quant_offset"] = qo.to(DEV)
    y, s = torch.ops.npu.npu_dequant_swiglu_quant(x.to(DEV), **kw)
    wy, wsc = G.dequant_swiglu_quant(x.numpy(), ws.numpy(), act.numpy(), bias.numpy(), qs.numpy(),
                                     counts.numpy() if grouped else None, left, quant_mode,
                                     None if qo is None else qo.numpy(), swiglu_mode=1, clamp_limit=6.0,
                                     glu_alpha=1.5, glu_bias=0.75)
    assert_int8_close(y.cpu().numpy(), wy)
    np.testing.assert_allclose(s.cpu().numpy(), wsc, rtol=1e-5, atol=0)


@pytest.mark.parametrize("seed", range(10))
def test_dynamic_quant_random(seed):
    """Seeded random npu_dynamic_quant shapes across the kernel variants (few and many rows, row widths
    that are and are not multiples of 8, up to 16 K columns), dtypes, and smooth scales with groups."""
    rng = np.random.default_rng(6000 + seed)
    g = gen(6000 + seed)
    rows = int(rng.choice([1, 3, 64, 700, 1500, 4100]))
    cols = int(rng.choice([8, 96, 1000, 2048, 7168, 7170, 16384]))
    dt = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(0, 3))]
    x = randn((rows, cols), g, dt)
    smooth = gidx = None
    if rng.random() < 0.5:
        ng = int(rng.integers(1, 5))
        smooth = uniform((ng, cols), g, 0.5, 2.0)
        ends = np.sort(rng.integers(0, rows + 1, ng))
        ends[-1] = rows
        gidx = torch.tensor(ends, dtype=torch.int64)
    print("case", dict(rows=rows, cols=cols, dt=str(dt), groups=None if gidx is None else gidx.tolist()), flush=True)
    _dq_check(x, smooth, gidx)


@pytest.mark.parametrize("seed", range(10))
def test_dequant_swiglu_quant_random(seed):
    """Seeded random npu_dequant_swiglu_quant: rows from 1 to thousands, n on and off the vector paths,
    groups (with empty ones and rows past the total), int32 / fp32 bias, quant_scale, both activate sides,
    dynamic and static quantisation, swiglu_mode 0 and 1."""
    rng = np.random.default_rng(7000 + seed)
    g = gen(7000 + seed)
    rows = int(rng.choice([1, 5, 128, 513, 2000]))
    n = int(rng.choice([4, 100, 512, 2048, 2049, 5632]))
    grouped = rng.random() < 0.5
    ng = int(rng.integers(1, 5)) if grouped else 1
    x = torch.randint(-100000, 100000, (rows, 2 * n), generator=g, dtype=torch.int32)
    ws = uniform((ng, 2 * n) if grouped else (2 * n,), g, 1e-4, 1e-3)
    act = uniform((rows,), g, 0.005, 0.05) if rng.random() < 0.7 else None
    bias = None
    r = rng.random()
    if r < 0.3:
        bias = torch.randint(-1000, 1000, (ng, 2 * n) if grouped else (2 * n,), generator=g, dtype=torch.int32)
    elif r < 0.5:
        bias = uniform((ng, 2 * n) if grouped else (2 * n,), g, -0.5, 0.5)
    qmode = int(rng.integers(0, 2))
    qs = uniform((ng, n) if grouped else (n,), g, 0.5, 2.0) if (qmode == 0 or rng.random() < 0.5) else None
    qo = uniform((ng, n) if grouped else (n,), g, -1.0, 1.0) if (qmode == 0 and rng.random() < 0.5) else None
    gidx = torch.tensor(rng.integers(0, rows // max(ng, 1) + 2, ng), dtype=torch.int64) if grouped else None
    left = bool(rng.integers(0, 2))
    smode = int(rng.integers(0, 2))
    case = dict(rows=rows, n=n, ng=ng, grouped=grouped, qmode=qmode, left=left, smode=smode,
                bias=None if bias is None else str(bias.dtype))
    print("case", case, flush=True)
    y, s = torch.ops.npu.npu_dequant_swiglu_quant(
        x.to(DEV), weight_scale=ws.to(DEV), activation_scale=None if act is None else act.to(DEV),
        bias=None if bias is None else bias.to(DEV), quant_scale=None if qs is None else qs.to(DEV),
        quant_offset=None if qo is None else qo.to(DEV), group_index=None if gidx is None else gidx.to(DEV),
        activate_left=left, quant_mode=qmode, swiglu_mode=smode)
    wy, wsc = G.dequant_swiglu_quant(x.numpy(), ws.numpy(), None if act is None else act.numpy(),
                                     None if bias is None else bias.numpy(), None if qs is None else qs.numpy(),
                                     None if gidx is None else gidx.numpy(), left, qmode,
                                     None if qo is None else qo.numpy(), swiglu_mode=smode)
    assert_int8_close(y.cpu().numpy(), wy)
    np.testing.assert_allclose(s.cpu().numpy(), wsc, rtol=1e-5, atol=1e-30, err_msg=str(case))
