"""GPU parity of the compiled graph's routing -> grouped GEMM fusion: tai::moe_init_routing_v2_rows
against npu_moe_init_routing_v2(quant_mode=1), and tai::grouped_matmul_gather against
npu_grouped_matmul over the materialised rows, bit for bit, on every GEMM path (mixed [K, N] tiles,
[N, K] tiles, the small-tile and generic kernels)."""
import pytest
import torch

import torchair_amd  # noqa: F401
from tests.helpers import gen

pytestmark = pytest.mark.gpu
DEV = "cuda"
npu, tai = torch.ops.npu, torch.ops.tai


def _route(t, h, e, k, g, active=None, row_idx_type=0, rng=None):
    x = torch.randn(t, h, generator=g).to(torch.bfloat16).to(DEV)
    idx = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(t)]).to(torch.int32).to(DEV)
    kw = dict(active_num=active if active is not None else t * k, expert_num=e, expert_tokens_num_type=1,
              row_idx_type=row_idx_type)
    if rng:
        kw["active_expert_range"] = rng
    want = npu.npu_moe_init_routing_v2(x, idx, expert_tokens_num_flag=True, quant_mode=1, **kw)
    got = tai.moe_init_routing_v2_rows(x, idx, **kw)
    return x, idx, want, got


@pytest.mark.parametrize("row_idx_type", [0, 1])
@pytest.mark.parametrize("active,rng", [(None, None), (150, None), (None, [2, 13])])
def test_routing_rows_equal_the_materialised_routing(row_idx_type, active, rng):
    g = gen(60)
    x, idx, (ex, ri, tok, es), (q, a_rows, ri2, tok2, es2) = _route(64, 512, 16, 4, g, active, row_idx_type, rng)
    assert torch.equal(ri, ri2) and torch.equal(tok, tok2) and torch.equal(es, es2)
    total = int(tok.sum())
    assert a_rows.shape[0] == ex.shape[0]
    assert torch.equal(q[a_rows[:total].long()], ex[:total])
    assert not ex[total:].any() and not a_rows[total:].any()
    wq, ws = npu.npu_dynamic_quant(x)
    assert torch.equal(q, wq)


@pytest.mark.parametrize("k,n,layout,out", [(512, 1024, "KN", "int32"), (512, 1024, "KN", "bf16"),
                                            (256, 384, "NK", "bf16"), (256, 200, "KN", "fp32"),
                                            (40, 48, "KN", "int32")])
def test_grouped_matmul_gather_equals_grouped_matmul(k, n, layout, out):
    g = gen(61)
    e = 16
    x, idx, (ex, ri, tok, es), (q, a_rows, *_ ) = _route(200, k, e, 3, g, active=520)
    w = torch.randint(-127, 128, (e, k, n), generator=g, dtype=torch.int8)
    wd = w.to(DEV) if layout == "KN" else w.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
    od = {"int32": torch.int32, "bf16": torch.bfloat16, "fp32": torch.float32}[out]
    kw = {}
    if out != "int32":
        kw = dict(scale=(torch.rand(e, n, generator=g) * 0.01 + 1e-3).to(DEV), per_token_scale=es)
    want = npu.npu_grouped_matmul([ex], [wd], group_list=tok, split_item=3, group_type=0, group_list_type=1,
                                  output_dtype=od, **{k_: [v] for k_, v in kw.items()})[0]
    got = tai.grouped_matmul_gather(q, a_rows, wd, tok, group_list_type=1, output_dtype=od, **kw)
    assert got.dtype == od and got.shape == want.shape
    assert torch.equal(got, want)


@pytest.mark.parametrize("layout,n", [("KN", 1024), ("KN", 512), ("NK", 512)])
def test_swiglu_quant_gather_equals_the_fused_op_on_materialised_rows(layout, n):
    g = gen(63)
    e, k = 16, 512
    x, idx, (ex, ri, tok, es), (q, a_rows, *_) = _route(200, k, e, 3, g, active=520)
    w = torch.randint(-127, 128, (e, k, n), generator=g, dtype=torch.int8)
    wd = w.to(DEV) if layout == "KN" else w.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
    ws = (torch.rand(e, n, generator=g) * 0.01 + 1e-3).to(DEV)
    y, s = npu.npu_grouped_matmul_swiglu_quant_v2(ex, [wd], [ws], es, tok, group_list_type=1)
    y2, s2 = tai.grouped_matmul_swiglu_quant_gather(q, a_rows, wd, ws, es, tok, group_list_type=1)
    assert torch.equal(y, y2) and torch.equal(s, s2)


def test_compiled_moe_block_uses_the_gather_and_matches_eager():
    from torchair_amd import CompilerConfig, get_npu_backend
    from torchair_amd.patterns import stats
    g = gen(62)
    t, h, e, k, i = 256, 1024, 32, 4, 512
    x = torch.randn(t, h, generator=g).to(torch.bfloat16).to(DEV)
    logits = torch.randn(t, e, generator=g).to(DEV)
    w = torch.randint(-127, 128, (e, h, 2 * i), generator=g, dtype=torch.int8).to(DEV)
    ws = (torch.rand(e, 2 * i, generator=g) * 0.01 + 1e-3).to(DEV)

    def block(x, logits):
        y, idx, _ = npu.npu_moe_gating_top_k(logits, k, k_group=1, group_count=1, norm_type=1)
        ex, ri, tok, _ = npu.npu_moe_init_routing_v2(x, idx, active_num=t * k, expert_num=e, expert_tokens_num_type=1,
                                                     expert_tokens_num_flag=True)
        q, s = npu.npu_dynamic_quant(ex)
        acc = npu.npu_grouped_matmul([q], [w], group_list=tok, split_item=3, group_type=0, group_list_type=1,
                                     output_dtype=torch.int32)[0]
        return npu.npu_dequant_swiglu_quant(acc, weight_scale=ws, activation_scale=s, group_index=tok,
                                            activate_left=True, quant_mode=1)

    cfg = CompilerConfig()
    cfg.mode = "reduce-overhead"
    before = stats["routing_grouped_matmul"]
    before_swiglu = stats["gather_dequant_swiglu_quant"]
    fn = torch.compile(block, backend=get_npu_backend(compiler_config=cfg), fullgraph=True)
    want = block(x, logits)
    for _ in range(3):  # capture, then replays
        got = fn(x, logits)
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert torch.equal(a, b)
    assert stats["routing_grouped_matmul"] == before + 1
    assert stats["gather_dequant_swiglu_quant"] == before_swiglu + 1
