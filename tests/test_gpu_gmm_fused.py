"""GPU parity: npu_grouped_matmul_swiglu_quant_v2 and npu_grouped_matmul_finalize_routing against the
CPU oracle and against the unfused GPU compositions they replace."""
import numpy as np
import pytest
import torch

import torchair_amd  # noqa: F401
from oracle import golden as G
from tests.helpers import assert_close, assert_int8_close, f32np, gen, rand_i8, uniform

pytestmark = pytest.mark.gpu
DEV = "cuda"
npu = torch.ops.npu


def _case(g, counts, k, n, m=None):
    e = len(counts)
    m = int(sum(counts)) if m is None else m
    x = rand_i8((m, k), g)
    w = rand_i8((e, k, n), g)
    ws = uniform((e, n), g, 1e-3, 1e-2)
    xs = uniform((m,), g, 1e-3, 1e-2)
    return x, w, ws, xs, torch.tensor(counts, dtype=torch.int64)


@pytest.mark.parametrize("layout", ["KN", "NK"])
@pytest.mark.parametrize("counts,k,n,extra", [([5, 0, 300, 17], 256, 512, 3), ([1, 1], 64, 1024, 0),
                                              ([128] * 6, 512, 1536, 0)])
def test_swiglu_quant_v2_vs_oracle(layout, counts, k, n, extra):
    g = gen(11)
    x, w, ws, xs, cnt = _case(g, counts, k, n, int(sum(counts)) + extra)
    wd = w.to(DEV) if layout == "KN" else w.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
    if layout == "NK" and (n // 2) % 128:
        pytest.skip("the [N, K] tiles cover 128 output columns")
    y, s = npu.npu_grouped_matmul_swiglu_quant_v2(x.to(DEV), [wd], [ws.to(DEV)], xs.to(DEV), cnt.to(DEV),
                                                  group_list_type=1)
    wy, wsc = G.grouped_matmul_swiglu_quant(x.numpy(), w.numpy(), ws.numpy(), xs.numpy(), cnt.numpy(), 1)
    assert y.shape == (x.shape[0], n // 2) and s.shape == (x.shape[0],)
    assert_int8_close(y.cpu().numpy(), wy)
    np.testing.assert_allclose(s.cpu().numpy(), wsc, rtol=1e-5, atol=0)


def test_swiglu_quant_v2_equals_unfused_gpu_path_cfg4_slice():
    # 16 experts of the config-4 gate_up shape: fused == grouped_matmul(int32) + dequant_swiglu_quant, bit for bit
    g = gen(12)
    counts = torch.randint(0, 300, (16,), generator=g).tolist()
    x, w, ws, xs, cnt = _case(g, counts, 7168, 4096)
    xd, wd, wsd, xsd, cd = x.to(DEV), w.to(DEV), ws.to(DEV), xs.to(DEV), cnt.to(DEV)
    y, s = npu.npu_grouped_matmul_swiglu_quant_v2(xd, [wd], [wsd], xsd, cd, group_list_type=1)
    acc = npu.npu_grouped_matmul([xd], [wd], group_list=cd, split_item=3, group_type=0, group_list_type=1,
                                 output_dtype=torch.int32)[0]
    y2, s2 = npu.npu_dequant_swiglu_quant(acc, weight_scale=wsd, activation_scale=xsd, group_index=cd,
                                          activate_left=True, quant_mode=1)
    assert torch.equal(y, y2) and torch.equal(s, s2)


@pytest.mark.parametrize("layout", ["KN", "NK"])
def test_finalize_routing_vs_oracle(layout):
    g = gen(13)
    t, kk, e, k, n = 96, 4, 6, 256, 384
    idx = torch.stack([torch.randperm(e, generator=g)[:kk] for _ in range(t)]).to(torch.int32)
    order = torch.argsort(idx.reshape(-1).to(torch.int64), stable=True)
    row_index = (order // kk).to(torch.int64)  # expanded row -> token
    counts = torch.bincount(idx.reshape(-1).to(torch.int64), minlength=e)
    x, w, sc, pts, _ = _case(g, counts.tolist(), k, n)
    logit = uniform((t * kk,), g, 0.0, 1.0)
    shared = torch.randn(10, n, generator=g).to(torch.bfloat16)
    wd = w.to(DEV) if layout == "KN" else w.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
    y = npu.npu_grouped_matmul_finalize_routing(x.to(DEV), wd, counts.to(DEV), scale=sc.to(DEV),
                                                pertoken_scale=pts.to(DEV), shared_input=shared.to(DEV),
                                                logit=logit.to(DEV), row_index=row_index.to(DEV),
                                                shared_input_weight=0.5, shared_input_offset=7, output_bs=t,
                                                group_list_type=1)
    want = G.grouped_matmul_finalize_routing(x.numpy(), w.numpy(), counts.numpy(), 1, sc.numpy(), pts.numpy(), None,
                                             logit.numpy(), row_index.numpy(), f32np(shared), 0.5, 7, t)
    assert y.dtype == torch.float32 and y.shape == (t, n)
    assert_close(y.cpu().numpy(), want)
    # deterministic: a second call gives identical bits
    y2 = npu.npu_grouped_matmul_finalize_routing(x.to(DEV), wd, counts.to(DEV), scale=sc.to(DEV),
                                                 pertoken_scale=pts.to(DEV), shared_input=shared.to(DEV),
                                                 logit=logit.to(DEV), row_index=row_index.to(DEV),
                                                 shared_input_weight=0.5, shared_input_offset=7, output_bs=t,
                                                 group_list_type=1)
    assert torch.equal(y, y2)


def test_finalize_routing_on_the_moe_routing_path():
    # routing from the GPU gating / init_routing ops; the fused op against the fp32 oracle, and the
    # unfused grouped_matmul(bf16) + moe_finalize_routing tail as a wiring check at bf16 precision
    g = gen(14)
    t, kk, e, k, n = 256, 8, 32, 512, 1024
    logits = torch.randn(t, e, generator=g)
    y_w, idx, _ = npu.npu_moe_gating_top_k(logits.to(DEV), kk, k_group=1, group_count=1, norm_type=1)
    xs = torch.randn(t, k, generator=g).to(torch.bfloat16).to(DEV)
    ex, ri, counts, _ = npu.npu_moe_init_routing_v2(xs, idx, active_num=t * kk, expert_num=e,
                                                    expert_tokens_num_type=1, expert_tokens_num_flag=True,
                                                    row_idx_type=0)
    q, s = npu.npu_dynamic_quant(ex)
    w = rand_i8((e, k, n), g).to(DEV)
    sc = uniform((e, n), g, 1e-3, 1e-2).to(DEV)
    # expanded row i holds routing slot p with ri[p] = i: token p // k, weight y_w[p]
    inv = torch.empty_like(ri)
    inv[ri.to(torch.int64)] = torch.arange(ri.numel(), device=DEV, dtype=ri.dtype)
    slot = inv.to(torch.int64)
    logit = y_w.reshape(-1)[slot].float()
    fused = npu.npu_grouped_matmul_finalize_routing(q, w, counts, scale=sc, pertoken_scale=s, logit=logit,
                                                    row_index=slot // kk, output_bs=t, group_list_type=1)
    want = G.grouped_matmul_finalize_routing(q.cpu().numpy(), w.cpu().numpy(), counts.cpu().numpy(), 1,
                                             sc.cpu().numpy(), s.cpu().numpy(), None, logit.cpu().numpy(),
                                             (slot // kk).cpu().numpy(), None, 1.0, 0, t)
    assert_close(fused.cpu().numpy(), want)
    out = npu.npu_grouped_matmul([q], [w], scale=[sc], per_token_scale=[s], group_list=counts, split_item=3,
                                 group_type=0, group_list_type=1, output_dtype=torch.bfloat16)[0]
    ref = npu.npu_moe_finalize_routing(out, None, None, None, y_w, ri, idx, drop_pad_mode=2)
    # bf16 rounding of the 8 rows and of the output: errors scale with the terms, not their sum
    np.testing.assert_allclose(ref.float().cpu().numpy(), want, rtol=3e-2, atol=0.15)


def test_swiglu_packed_weight_layout_and_cache():
    """[E, K, N] weights are packed once (gate / up interleaved in 64-column blocks) and the packed copy
    is rebuilt when the weight is written in place; results equal the unpacked layout bit for bit."""
    from torchair_amd import _gmm_fused as F
    g = gen(13)
    counts = [70, 0, 200, 9]
    x, w, ws, xs, cnt = _case(g, counts, 256, 1024)
    xd, wd, wsd, xsd, cd = x.to(DEV), w.to(DEV), ws.to(DEV), xs.to(DEV), cnt.to(DEV)
    p = F._swiglu_packed(wd)
    e, k, n = w.shape
    want = w.view(e, k, 2, n // 128, 64).permute(0, 1, 3, 2, 4).reshape(e, k, n)
    assert torch.equal(p.cpu(), want)
    assert F._swiglu_packed(wd) is p  # cached
    y, s = npu.npu_grouped_matmul_swiglu_quant_v2(xd, [wd], [wsd], xsd, cd, group_list_type=1)
    # the unpacked [K, N] layout through the C ABI
    from torchair_amd import _lib
    nbytes = _lib.query("tai_grouped_matmul_swiglu_quant_workspace_size", x.shape[0], n, e)
    wsp = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    y0 = torch.empty_like(y)
    s0 = torch.empty_like(s)
    _lib.call("tai_grouped_matmul_swiglu_quant", xd.data_ptr(), wd.data_ptr(), x.shape[0], k, n, e, _lib.LAYOUT_KN,
              cd.data_ptr(), 1, wsd.data_ptr(), xsd.data_ptr(), y0.data_ptr(), s0.data_ptr(), wsp.data_ptr(), nbytes,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(y, y0) and torch.equal(s, s0)
    wd[1:3] = -wd[1:3]  # in-place write: the packed copy is stale
    p2 = F._swiglu_packed(wd)
    assert torch.equal(p2.cpu(), wd.cpu().view(e, k, 2, n // 128, 64).permute(0, 1, 3, 2, 4).reshape(e, k, n))
    y3, _ = npu.npu_grouped_matmul_swiglu_quant_v2(xd, [wd], [wsd], xsd, cd, group_list_type=1)
    wy, _ = G.grouped_matmul_swiglu_quant(x.numpy(), wd.cpu().numpy(), ws.numpy(), xs.numpy(), cnt.numpy(), 1)
    assert_int8_close(y3.cpu().numpy(), wy)


@pytest.mark.parametrize("bias_kind,smooth_kind", [("int32", "per_group"), ("fp32", "shared"), (None, "per_group"),
                                                   ("int32", None)])
def test_swiglu_quant_v2_smooth_scale_and_bias(bias_kind, smooth_kind):
    """smooth_scale and bias: the grouped GEMM's int32 accumulators, then dequant_swiglu_quant with the
    bias (int32 before, fp32 after the dequantisation) and the smooth scale as its quant_scale."""
    g = gen(13)
    counts, k, n = [7, 0, 130, 33], 256, 512
    e = len(counts)
    x, w, ws, xs, cnt = _case(g, counts, k, n, int(sum(counts)) + 2)
    kw = {}
    bias = sm = None
    if bias_kind == "int32":
        bias = torch.randint(-5000, 5000, (e, n), generator=g, dtype=torch.int32)
    elif bias_kind == "fp32":
        bias = uniform((e, n), g, -0.5, 0.5)
    if smooth_kind == "per_group":
        sm = uniform((e, n // 2), g, 0.5, 2.0)
    elif smooth_kind == "shared":
        sm = uniform((n // 2,), g, 0.5, 2.0)
    if bias is not None:
        kw["bias"] = bias.to(DEV)
    if sm is not None:
        kw["smooth_scale"] = sm.to(DEV)
    y, s = npu.npu_grouped_matmul_swiglu_quant_v2(x.to(DEV), [w.to(DEV)], [ws.to(DEV)], xs.to(DEV),
                                                  torch.cumsum(cnt, 0).to(DEV), group_list_type=0, **kw)
    acc = G.grouped_matmul(x.numpy(), w.numpy(), cnt.numpy(), 1, out_dtype="int32")
    smn = None if sm is None else np.broadcast_to(sm.numpy().reshape(-1, n // 2), (e, n // 2))
    wy, wsc = G.dequant_swiglu_quant(acc, ws.numpy(), xs.numpy(), None if bias is None else bias.numpy(), smn,
                                     cnt.numpy(), activate_left=True)
    assert_int8_close(y.cpu().numpy(), wy)
    np.testing.assert_allclose(s.cpu().numpy(), wsc, rtol=1e-5, atol=0)


_EDGE = [0, 1, 31, 32, 33, 64, 127, 128, 129, 255, 256, 257, 300]


@pytest.mark.parametrize("seed", range(8))
def test_swiglu_quant_v2_random(seed):
    """Seeded random npu_grouped_matmul_swiglu_quant_v2: group sizes at the tile boundaries (empty groups,
    the 128- and 256-row tiles), rows past the total, K, N and both weight layouts, count and cumsum lists."""
    rng = np.random.default_rng(10000 + seed)
    g = gen(10000 + seed)
    e = int(rng.integers(1, 8))
    counts = [int(rng.choice(_EDGE)) for _ in range(e)]
    layout = "KN" if rng.random() < 0.6 else "NK"
    n = int(rng.choice([512, 1024, 1536]))
    k = 128 * int(rng.integers(1, 12))
    extra = int(rng.integers(0, 20))
    list_type = int(rng.integers(0, 2))
    x, w, ws, xs, cnt = _case(g, counts, k, n, sum(counts) + extra)
    wd = w.to(DEV) if layout == "KN" else w.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
    gl = cnt if list_type == 1 else torch.cumsum(cnt, 0)
    print("case", dict(counts=counts, layout=layout, n=n, k=k, extra=extra, list_type=list_type), flush=True)
    y, s = npu.npu_grouped_matmul_swiglu_quant_v2(x.to(DEV), [wd], [ws.to(DEV)], xs.to(DEV), gl.to(DEV),
                                                  group_list_type=list_type)
    wy, wsc = G.grouped_matmul_swiglu_quant(x.numpy(), w.numpy(), ws.numpy(), xs.numpy(), cnt.numpy(), 1)
    assert_int8_close(y.cpu().numpy(), wy)
    np.testing.assert_allclose(s.cpu().numpy(), wsc, rtol=1e-5, atol=0)


@pytest.mark.parametrize("seed", range(6))
def test_finalize_routing_random(seed):
    """Seeded random npu_grouped_matmul_finalize_routing: tokens, top-k, experts (some empty), K, N, both
    weight layouts, with and without the shared input."""
    rng = np.random.default_rng(10100 + seed)
    g = gen(10100 + seed)
    t, kk = int(rng.integers(1, 200)), int(rng.integers(1, 9))
    e = int(rng.integers(kk, 3 * kk + 2))
    k, n = 64 * int(rng.integers(1, 12)), int(rng.choice([128, 256, 384, 512, 1024]))
    layout = "KN" if rng.random() < 0.5 else "NK"
    idx = torch.stack([torch.randperm(e, generator=g)[:kk] for _ in range(t)]).to(torch.int32)
    order = torch.argsort(idx.reshape(-1).to(torch.int64), stable=True)
    row_index = (order // kk).to(torch.int64)
    counts = torch.bincount(idx.reshape(-1).to(torch.int64), minlength=e)
    x, w, sc, pts, _ = _case(g, counts.tolist(), k, n)
    logit = uniform((t * kk,), g, 0.0, 1.0)
    wd = w.to(DEV) if layout == "KN" else w.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
    kw = {}
    shared = None
    if rng.random() < 0.5:
        off = int(rng.integers(0, 5))
        shared = torch.randn(max(t - off, 1), n, generator=g).to(torch.bfloat16)
        kw = dict(shared_input=shared.to(DEV), shared_input_weight=0.25, shared_input_offset=off)
    print("case", dict(t=t, kk=kk, e=e, k=k, n=n, layout=layout, shared=shared is not None), flush=True)
    y = npu.npu_grouped_matmul_finalize_routing(x.to(DEV), wd, counts.to(DEV), scale=sc.to(DEV),
                                                pertoken_scale=pts.to(DEV), logit=logit.to(DEV),
                                                row_index=row_index.to(DEV), output_bs=t, group_list_type=1, **kw)
    want = G.grouped_matmul_finalize_routing(x.numpy(), w.numpy(), counts.numpy(), 1, sc.numpy(), pts.numpy(), None,
                                             logit.numpy(), row_index.numpy(),
                                             None if shared is None else f32np(shared),
                                             kw.get("shared_input_weight", 1.0), kw.get("shared_input_offset", 0), t)
    assert_close(y.cpu().numpy(), want)
