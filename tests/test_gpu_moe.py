"""GPU parity: MoE gating top-k, init routing (v2 and legacy) and finalize routing."""
import numpy as np
import pytest
import torch

import torchair_amd  # noqa: F401
from oracle import golden as G
from tests.helpers import assert_close, assert_int8_close, f32np, gen, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _gate_check(x, k, bias=None, **kw):
    y, idx, out = torch.ops.npu.npu_moe_gating_top_k(x.to(DEV), k, bias=None if bias is None else bias.to(DEV), **kw)
    name = {torch.float32: "fp32", torch.bfloat16: "bf16", torch.float16: "fp16"}[x.dtype]
    wy, widx, wout = G.moe_gating_top_k(f32np(x), k, None if bias is None else f32np(bias),
                                        kw.get("k_group", 1), kw.get("group_count", 1),
                                        kw.get("group_select_mode", 0), kw.get("renorm", 0), kw.get("norm_type", 0),
                                        kw.get("out_flag", False), kw.get("routed_scaling_factor", 1.0),
                                        kw.get("eps", 1e-20), name)
    np.testing.assert_array_equal(idx.cpu().numpy(), widx)
    np.testing.assert_allclose(f32np(y), wy, rtol=1e-6, atol=1e-7)
    if kw.get("out_flag", False):
        np.testing.assert_allclose(out.cpu().numpy(), wout, rtol=1e-6, atol=1e-7)
    return idx


def test_gating_cfg4_deepseek():
    g = gen(30)
    x = torch.randn(4096, 256, generator=g)
    bias = torch.randn(256, generator=g) * 0.1
    _gate_check(x, 8, bias, k_group=4, group_count=8, group_select_mode=1, norm_type=1, out_flag=True,
                routed_scaling_factor=2.5)


def test_gating_variants():
    g = gen(31)
    x = torch.randn(513, 64, generator=g)
    _gate_check(x, 6)  # softmax, plain top-k
    _gate_check(x, 4, k_group=2, group_count=4, group_select_mode=0, norm_type=1)
    _gate_check(x.to(torch.bfloat16), 8, torch.randn(64, generator=g).to(torch.bfloat16), k_group=3, group_count=8,
                group_select_mode=1, norm_type=1)


def test_gating_ties_pick_lower_index():
    x = torch.zeros(3, 32)
    x[1, 5] = x[1, 9] = x[1, 30] = 1.0
    idx = _gate_check(x, 4, k_group=2, group_count=4, group_select_mode=1, norm_type=1)
    assert idx.cpu()[0].tolist() == [0, 1, 2, 3]


@pytest.mark.parametrize("groups,k_group,mode", [(8, 4, 1), (8, 3, 0), (1, 1, 1), (8, 8, 1)])
def test_gating_256_experts_register_path(groups, k_group, mode):
    """E = 256 with sigmoid scores takes the register-resident kernel (8 groups of 32 or no groups): the
    oracle's choices and weights, including rows with tied scores, tied group scores and a bf16 input."""
    g = gen(32)
    x = torch.randn(1037, 256, generator=g)
    x[3] = 0.0                      # every score tied
    x[4, ::7] = 2.0                 # ties across groups
    x[5, 32:64] = 1.5               # one group of equal maxima (top-2 = 2 * max)
    bias = torch.randn(256, generator=g) * 0.1
    _gate_check(x, 8, bias, k_group=k_group, group_count=groups, group_select_mode=mode, norm_type=1, out_flag=True,
                routed_scaling_factor=2.5)
    _gate_check(x.to(torch.bfloat16), 6, bias.to(torch.bfloat16), k_group=k_group, group_count=groups,
                group_select_mode=mode, norm_type=1)


def _routing_inputs(t, h, e, k, g):
    x = randn((t, h), g)
    logits = torch.randn(t, e, generator=g)
    idx = torch.argsort(torch.rand(t, e, generator=g), dim=1)[:, :k].to(torch.int32)
    del logits
    return x, idx


@pytest.mark.parametrize("row_idx_type", [0, 1])
@pytest.mark.parametrize("tokens_type", [0, 1])
def test_init_routing_v2_cfg4(row_idx_type, tokens_type):
    g = gen(32)
    t, h, e, k = 4096, 7168, 256, 8
    x, idx = _routing_inputs(t, h, e, k, g)
    ex, ri, tok, es = torch.ops.npu.npu_moe_init_routing_v2(
        x.to(DEV), idx.to(DEV), active_num=t * k, expert_num=e, expert_tokens_num_type=tokens_type,
        expert_tokens_num_flag=True, row_idx_type=row_idx_type)
    wex, wri, wtok, _ = G.moe_init_routing_v2(f32np(x), idx.numpy(), None, t * k, 0, e, tokens_type, row_idx_type)
    np.testing.assert_array_equal(ri.cpu().numpy(), wri)
    np.testing.assert_array_equal(tok.cpu().numpy(), wtok)
    np.testing.assert_array_equal(f32np(ex), wex)


def test_init_routing_v2_range_active_and_scale():
    g = gen(33)
    t, h, e, k = 333, 96, 32, 4
    x, idx = _routing_inputs(t, h, e, k, g)
    scale = torch.rand(t, generator=g)
    ex, ri, tok, es = torch.ops.npu.npu_moe_init_routing_v2(
        x.to(DEV), idx.to(DEV), scale=scale.to(DEV), active_num=700, expert_num=e, active_expert_range=[4, 20],
        expert_tokens_num_type=1, row_idx_type=0)
    wex, wri, wtok, wes = G.moe_init_routing_v2(f32np(x), idx.numpy(), scale.numpy(), 700, 4, 20, 1, 0)
    np.testing.assert_array_equal(ri.cpu().numpy(), wri)
    np.testing.assert_array_equal(tok.cpu().numpy(), wtok)
    np.testing.assert_array_equal(f32np(ex), wex)
    np.testing.assert_array_equal(es.cpu().numpy(), wes)


def test_init_routing_v2_dynamic_quant_cfg4():
    # quant_mode 1: int8 expanded rows and their per-row scales, bit for bit the npu_dynamic_quant of
    # the gathered bf16 rows
    g = gen(35)
    t, h, e, k = 4096, 7168, 256, 8
    x, idx = _routing_inputs(t, h, e, k, g)
    ex, ri, tok, es = torch.ops.npu.npu_moe_init_routing_v2(
        x.to(DEV), idx.to(DEV), active_num=t * k, expert_num=e, expert_tokens_num_type=1,
        expert_tokens_num_flag=True, quant_mode=1)
    assert ex.dtype == torch.int8 and es.shape == (t * k,)
    wex, wri, wtok, _ = G.moe_init_routing_v2(f32np(x), idx.numpy(), None, t * k, 0, e, 1, 0)
    wq, ws = G.dynamic_quant(wex)
    np.testing.assert_array_equal(ri.cpu().numpy(), wri)
    np.testing.assert_array_equal(tok.cpu().numpy(), wtok)
    np.testing.assert_array_equal(ex.cpu().numpy(), wq)
    np.testing.assert_array_equal(es.cpu().numpy(), ws)
    # and the same as the unfused pair of ops
    ex2, _, _, _ = torch.ops.npu.npu_moe_init_routing_v2(x.to(DEV), idx.to(DEV), active_num=t * k, expert_num=e,
                                                         expert_tokens_num_type=1, expert_tokens_num_flag=True)
    q2, s2 = torch.ops.npu.npu_dynamic_quant(ex2)
    assert torch.equal(q2, ex) and torch.equal(s2, es)


def test_init_routing_legacy():
    g = gen(34)
    t, h, k = 250, 64, 3
    x = randn((t, h), g, torch.float32)
    idx = torch.randint(0, 10, (t, k), generator=g, dtype=torch.int32)
    row = torch.arange(t * k, dtype=torch.int32).view(k, t).t().contiguous()
    for active in (t, 100):
        ex, ri, ei = torch.ops.npu.npu_moe_init_routing(x.to(DEV), row.to(DEV), idx.to(DEV), active)
        wex, wri, wei = G.moe_init_routing(x.numpy(), row.numpy(), idx.numpy(), active)
        np.testing.assert_array_equal(ri.cpu().numpy(), wri)
        np.testing.assert_array_equal(ei.cpu().numpy(), wei)
        np.testing.assert_array_equal(ex.cpu().numpy(), wex)


def test_finalize_cfg4():
    g = gen(35)
    t, h, k = 4096, 7168, 8
    n = t * k
    expanded = randn((n, h), g)
    perm = torch.randperm(n, generator=g).to(torch.int32)
    scales = torch.rand(t, k, generator=g)
    y = torch.ops.npu.npu_moe_finalize_routing(expanded.to(DEV), None, None, None, scales.to(DEV), perm.to(DEV), None,
                                               drop_pad_mode=2)
    want = G.moe_finalize_routing(f32np(expanded), None, None, None, scales.numpy(), perm.numpy(), None, 2, "bf16")
    assert_close(f32np(y), want)


@pytest.mark.parametrize("dtype,name", [(torch.bfloat16, "bf16"), (torch.float16, "fp16"), (torch.float32, "fp32")])
def test_finalize_declared_cases(dtype, name):
    """Shapes of the reference's declared cases (npu_moe_finalize_routing.py:4-20)."""
    g = gen(36)
    ex = randn((24, 7), g, dtype)
    s1, s2, bias = randn((12, 7), g, dtype), randn((12, 7), g, dtype), randn((3, 7), g, dtype)
    scales = randn((12, 2), g, dtype)
    row = torch.arange(24, dtype=torch.int32)
    exp = torch.randint(0, 3, (12, 2), generator=g, dtype=torch.int32)
    for args in ((s1, s2, bias, scales), (s1, None, bias, scales), (None, None, None, scales)):
        a1, a2, b, sc = args
        y = torch.ops.npu.npu_moe_finalize_routing(ex.to(DEV), *(None if v is None else v.to(DEV) for v in (a1, a2, b, sc)),
                                                   row.to(DEV), exp.to(DEV), drop_pad_mode=0)
        want = G.moe_finalize_routing(f32np(ex), *(None if v is None else f32np(v) for v in (a1, a2, b, sc)),
                                      row.numpy(), exp.numpy(), 0, name)
        assert_close(f32np(y), want, rtol=2e-2, atol=2e-2)


def test_routing_round_trip():
    """finalize(init(x)) with weights summing to one returns x (token-major slots)."""
    g = gen(37)
    t, h, e, k = 1000, 256, 64, 8
    x, idx = _routing_inputs(t, h, e, k, g)
    ex, ri, tok, _ = torch.ops.npu.npu_moe_init_routing_v2(x.to(DEV), idx.to(DEV), expert_num=e)
    w = torch.full((t, k), 1.0 / k, device=DEV)
    y = torch.ops.npu.npu_moe_finalize_routing(ex, None, None, None, w, ri, idx.to(DEV), drop_pad_mode=2)
    assert_close(f32np(y), f32np(x))
    assert int(tok[-1]) == t * k


# ----------------------------------------------------------------------------- drop-pad, static / smooth quant
@pytest.mark.parametrize("cap", [1, 7, 64])
def test_init_routing_v2_drop_pad(cap):
    """drop_pad_mode 1: expert e owns rows [e * cap, (e + 1) * cap); slots past the capacity are dropped;
    unfilled rows are zero; the gathered per-token scale follows its row."""
    g = gen(34)
    t, h, e, k = 300, 64, 16, 4
    x, idx = _routing_inputs(t, h, e, k, g)
    scale = torch.rand(t, generator=g)
    ex, ri, tok, es = torch.ops.npu.npu_moe_init_routing_v2(
        x.to(DEV), idx.to(DEV), scale=scale.to(DEV), expert_capacity=cap, expert_num=e, drop_pad_mode=1,
        expert_tokens_num_type=1, expert_tokens_num_flag=True)
    wex, wri, wtok, wes = G.moe_init_routing_v2_droppad(f32np(x), idx.numpy(), cap, scale.numpy(), 0, e, 1)
    assert ex.shape == (e * cap, h)
    np.testing.assert_array_equal(ri.cpu().numpy(), wri)
    np.testing.assert_array_equal(tok.cpu().numpy(), wtok)
    np.testing.assert_array_equal(f32np(ex), wex)
    np.testing.assert_array_equal(es.cpu().numpy(), wes)


def test_init_routing_v2_drop_pad_dynamic_quant_and_range():
    """drop-pad with quant_mode 1 (no smooth scale) over an active expert range: the int8 rows and scales
    of npu_dynamic_quant's token rows, placed by the drop-pad rule."""
    g = gen(35)
    t, h, e, k, cap = 257, 128, 32, 8, 40
    x, idx = _routing_inputs(t, h, e, k, g)
    ex, ri, tok, es = torch.ops.npu.npu_moe_init_routing_v2(
        x.to(DEV), idx.to(DEV), expert_capacity=cap, expert_num=e, drop_pad_mode=1, quant_mode=1,
        active_expert_range=[3, 19], expert_tokens_num_type=0)
    q, s = G.dynamic_quant(f32np(x))
    wex, wri, wtok, wes = G.moe_init_routing_v2_droppad(q, idx.numpy(), cap, s, 3, 19, 0)
    np.testing.assert_array_equal(ri.cpu().numpy(), wri)
    np.testing.assert_array_equal(tok.cpu().numpy(), wtok)
    np.testing.assert_array_equal(ex.cpu().numpy(), wex)
    np.testing.assert_array_equal(es.cpu().numpy(), wes)


@pytest.mark.parametrize("drop_pad", [0, 1])
@pytest.mark.parametrize("shared", [False, True])
def test_init_routing_v2_dynamic_quant_smooth(drop_pad, shared):
    """quant_mode 1 with a smooth scale ([1, H] shared, or [E, H] per expert): each expanded row is x * smooth
    of its expert, quantised per row (int8 within 1 LSB on at most 0.1%, scales rtol 1e-6)."""
    g = gen(36)
    t, h, e, k, cap = 200, 256, 16, 4, 64
    x, idx = _routing_inputs(t, h, e, k, g)
    sm = torch.rand(1 if shared else e, h, generator=g) + 0.5
    ex, ri, tok, es = torch.ops.npu.npu_moe_init_routing_v2(
        x.to(DEV), idx.to(DEV), scale=sm.to(DEV), expert_capacity=cap, expert_num=e, drop_pad_mode=drop_pad,
        quant_mode=1, active_num=t * k, expert_tokens_num_type=1)
    if drop_pad:
        bex, wri, wtok, _ = G.moe_init_routing_v2_droppad(f32np(x), idx.numpy(), cap, None, 0, e, 1)
        ends = np.arange(1, e + 1) * cap
    else:
        bex, wri, wtok, _ = G.moe_init_routing_v2(f32np(x), idx.numpy(), None, t * k, 0, e, 1, 0)
        ends = np.cumsum(wtok)
    if shared:
        wq, ws = G.dynamic_quant(bex, sm.numpy().reshape(h))
    else:
        wq, ws = G.dynamic_quant(bex, sm.numpy(), group_index=ends)
    np.testing.assert_array_equal(ri.cpu().numpy(), wri)
    np.testing.assert_array_equal(tok.cpu().numpy(), wtok)
    assert_int8_close(ex.cpu().numpy(), wq)
    np.testing.assert_allclose(es.cpu().numpy(), ws, rtol=1e-6, atol=0)


@pytest.mark.parametrize("drop_pad", [0, 1])
@pytest.mark.parametrize("form", ["tensor", "expert_channel", "expert"])
def test_init_routing_v2_static_quant(drop_pad, form):
    """quant_mode 0: clamp(rint(x * scale + offset)) with per-tensor, per-expert or per-expert-and-channel
    scale and offset, bit for bit."""
    g = gen(37)
    t, h, e, k, cap = 150, 64, 8, 3, 80
    x, idx = _routing_inputs(t, h, e, k, g)
    shape = {"tensor": (1,), "expert_channel": (e, h), "expert": (e, 1)}[form]
    sc = torch.rand(shape, generator=g) * 40 + 10
    of = torch.rand(shape, generator=g) * 4 - 2
    ex, ri, tok, es = torch.ops.npu.npu_moe_init_routing_v2(
        x.to(DEV), idx.to(DEV), scale=sc.to(DEV), offset=of.to(DEV), expert_capacity=cap, expert_num=e,
        drop_pad_mode=drop_pad, quant_mode=0, expert_tokens_num_type=1)
    if drop_pad:
        bex, wri, wtok, _ = G.moe_init_routing_v2_droppad(f32np(x), idx.numpy(), cap, None, 0, e, 1)
        grp = np.arange(e * cap) // cap
    else:
        bex, wri, wtok, _ = G.moe_init_routing_v2(f32np(x), idx.numpy(), None, t * k, 0, e, 1, 0)
        grp = np.repeat(np.arange(e), wtok)
    assert ex.dtype == torch.int8 and es.numel() == 0
    np.testing.assert_array_equal(ri.cpu().numpy(), wri)
    np.testing.assert_array_equal(ex.cpu().numpy(), G.static_quant_rows(bex, sc.numpy(), of.numpy(), grp))


def test_moe_compute_expert_tokens():
    g = gen(33)
    for n, e in ((0, 16), (1, 1), (32768, 256), (1000, 64)):
        se = torch.sort(torch.randint(0, e + 2, (n,), generator=g)).values.to(torch.int32)  # ids past E too
        got = torch.ops.npu.npu_moe_compute_expert_tokens(se.to(DEV), e)
        assert got.dtype == torch.int32 and got.shape == (e,)
        np.testing.assert_array_equal(got.cpu().numpy(), G.moe_compute_expert_tokens(se.numpy(), e))


@pytest.mark.parametrize("seed", range(10))
def test_init_routing_v2_random(seed):
    """Seeded random routing bit-exact against the oracle: token and expert counts, top-k, the expert
    range, active_num, dropless or drop-pad with a capacity, gather or scatter row indices, counts or
    cumsum, with a per-token scale carried along (skewed routings included)."""
    rng = np.random.default_rng(4000 + seed)
    g = gen(4000 + seed)
    t, e = int(rng.integers(1, 700)), int(rng.choice([8, 16, 64, 256]))
    k = int(rng.integers(1, min(e, 8) + 1))
    h = 16 * int(rng.integers(1, 9))
    if rng.random() < 0.3:  # skewed: most slots on a few experts
        idx = torch.from_numpy(np.stack([rng.permutation(min(e, 2 * k))[:k] for _ in range(t)]).astype(np.int32))
    else:
        idx = torch.from_numpy(np.stack([rng.permutation(e)[:k] for _ in range(t)]).astype(np.int32))
    x = torch.randn(t, h, generator=g)
    scale = torch.rand(t, generator=g)
    lo = int(rng.integers(0, e // 2))
    hi = int(rng.integers(lo + 1, e + 1))
    tok_type = int(rng.integers(0, 2))
    case = dict(t=t, e=e, k=k, h=h, lo=lo, hi=hi, tok_type=tok_type)
    if rng.random() < 0.4:
        cap = int(rng.integers(1, 3 * t * k // e + 2))
        case["cap"] = cap
        print("case", case, flush=True)
        ex, ri, tok, es = torch.ops.npu.npu_moe_init_routing_v2(
            x.to(DEV), idx.to(DEV), scale=scale.to(DEV), expert_capacity=cap, expert_num=e, drop_pad_mode=1,
            active_expert_range=[lo, hi], expert_tokens_num_type=tok_type, expert_tokens_num_flag=True)
        wex, wri, wtok, wes = G.moe_init_routing_v2_droppad(f32np(x), idx.numpy(), cap, scale.numpy(), lo, hi,
                                                            tok_type)
    else:
        active = int(rng.integers(1, t * k + 1))
        row_type = int(rng.integers(0, 2))
        case.update(active=active, row_type=row_type)
        print("case", case, flush=True)
        ex, ri, tok, es = torch.ops.npu.npu_moe_init_routing_v2(
            x.to(DEV), idx.to(DEV), scale=scale.to(DEV), active_num=active, expert_num=e,
            active_expert_range=[lo, hi], expert_tokens_num_type=tok_type, row_idx_type=row_type)
        wex, wri, wtok, wes = G.moe_init_routing_v2(f32np(x), idx.numpy(), scale.numpy(), active, lo, hi, tok_type,
                                                    row_type)
    np.testing.assert_array_equal(ri.cpu().numpy(), wri, err_msg=str(case))
    np.testing.assert_array_equal(tok.cpu().numpy(), wtok, err_msg=str(case))
    np.testing.assert_array_equal(f32np(ex), wex, err_msg=str(case))
    np.testing.assert_array_equal(es.cpu().numpy(), wes, err_msg=str(case))


@pytest.mark.parametrize("seed", range(10))
def test_gating_top_k_random(seed):
    """Seeded random npu_moe_gating_top_k bit-exact (ids) against the oracle: expert and group counts
    (the 256-expert register kernel and the general one), k, k_group, group selection by max or top-2
    sum, sigmoid or softmax scores, with or without bias and the normalised-score output."""
    rng = np.random.default_rng(5000 + seed)
    g = gen(5000 + seed)
    e = int(rng.choice([16, 64, 128, 256, 256]))
    group_count = int(rng.choice([c for c in (1, 2, 4, 8) if e % c == 0 and e // c >= 2]))
    k_group = int(rng.integers(1, group_count + 1))
    per_group = e // group_count
    k = int(rng.integers(1, min(8, k_group * per_group) + 1))
    mode = int(rng.integers(0, 2))
    norm = int(rng.integers(0, 2))
    t = int(rng.integers(1, 500))
    x = torch.randn(t, e, generator=g)
    bias = torch.randn(e, generator=g) * 0.1 if rng.random() < 0.6 else None
    out_flag = bool(rng.integers(0, 2))
    rsf = float(rng.choice([1.0, 2.5]))
    case = dict(e=e, groups=group_count, k_group=k_group, k=k, mode=mode, norm=norm, t=t, bias=bias is not None)
    print("case", case, flush=True)
    y, idx, out = torch.ops.npu.npu_moe_gating_top_k(
        x.to(DEV), k, bias=None if bias is None else bias.to(DEV), k_group=k_group, group_count=group_count,
        group_select_mode=mode, renorm=0, norm_type=norm, out_flag=out_flag, routed_scaling_factor=rsf, eps=1e-20)
    wy, widx, wout = G.moe_gating_top_k(x.numpy(), k, None if bias is None else bias.numpy(), k_group, group_count,
                                        mode, 0, norm, out_flag, rsf, 1e-20)
    np.testing.assert_array_equal(idx.cpu().numpy(), widx, err_msg=str(case))
    np.testing.assert_allclose(y.cpu().numpy(), wy, rtol=1e-6, atol=1e-7, err_msg=str(case))
    if out_flag:
        np.testing.assert_allclose(out.cpu().numpy(), wout, rtol=1e-6, atol=1e-7, err_msg=str(case))


@pytest.mark.parametrize("seed", range(8))
def test_finalize_routing_random(seed):
    """Seeded random npu_moe_finalize_routing against the oracle: both slot conventions (drop_pad_mode 0,
    k-major; 2, token-major), dropped rows (-1), skip inputs, per-expert bias, scales absent or given,
    widths on and off the 16-byte path, bf16 / fp16 / fp32."""
    rng = np.random.default_rng(8000 + seed)
    g = gen(8000 + seed)
    t, k = int(rng.integers(1, 300)), int(rng.integers(1, 9))
    h = int(rng.choice([8, 64, 100, 7168]))
    e = int(rng.integers(2, 40))
    dt, name = [(torch.bfloat16, "bf16"), (torch.float16, "fp16"), (torch.float32, "fp32")][int(rng.integers(0, 3))]
    mode = int(rng.choice([0, 2]))
    n = t * k
    rows = n + int(rng.integers(0, 20))
    ex = randn((rows, h), g, dt)
    s2d = torch.randperm(rows, generator=g)[:n].to(torch.int32)
    s2d[torch.rand(n, generator=g) < 0.1] = -1  # dropped slots
    expert = torch.randint(0, e, (t, k), generator=g, dtype=torch.int32)
    skip1 = randn((t, h), g, dt) if rng.random() < 0.5 else None
    skip2 = randn((t, h), g, dt) if skip1 is not None and rng.random() < 0.5 else None
    bias = randn((e, h), g, dt) if rng.random() < 0.5 else None
    scales = torch.rand(t, k, generator=g).to(dt) if rng.random() < 0.8 else None
    case = dict(t=t, k=k, h=h, e=e, dt=name, mode=mode, skip1=skip1 is not None, skip2=skip2 is not None,
                bias=bias is not None, scales=scales is not None)
    print("case", case, flush=True)
    dv = lambda v: None if v is None else v.to(DEV)  # noqa: E731
    y = torch.ops.npu.npu_moe_finalize_routing(dv(ex), dv(skip1), dv(skip2), dv(bias), dv(scales), dv(s2d),
                                               dv(expert), drop_pad_mode=mode)
    npf = lambda v: None if v is None else f32np(v)  # noqa: E731
    want = G.moe_finalize_routing(f32np(ex), npf(skip1), npf(skip2), npf(bias), npf(scales), s2d.numpy(),
                                  expert.numpy(), mode, name)
    assert_close(f32np(y), want, rtol=2e-2, atol=2e-2)
