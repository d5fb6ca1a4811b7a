"""GPU parity of the config-4 MoE layer exactly as bench.py runs it: bench.MoeLayer's inputs
(seed 0), its gating-derived, skewed group list (0 to ~940 rows per expert, so up to 8 row
tiles share one weight slice) and its op sequence, checked stage by stage:
  gating ids and the routing permutation / counts bit-exact against the oracle; the quantised
  rows against the oracle on every row (+-1 LSB); the gate_up int32 accumulators exact against a float64 GPU
  product for EVERY live expert; dequant_swiglu_quant against the oracle on every row (+-1 LSB); the
  bf16 down projection at full shape against float64 for every live expert (rtol = atol = 1e-2);
  finalize against the oracle for every token; the hipGraph replay of the layer equal to eager."""
import numpy as np
import pytest
import torch

import bench
import torchair_amd  # noqa: F401
from oracle import golden as G
from tests.helpers import assert_close, assert_int8_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def layer():
    lay = bench.MoeLayer(torch, DEV)
    yield lay
    del lay
    torch.cuda.empty_cache()


def _stages(L):
    npu = torch.ops.npu
    y, idx, _ = npu.npu_moe_gating_top_k(L.logits, L.K, bias=L.bias, k_group=4, group_count=8, group_select_mode=1,
                                         renorm=0, norm_type=1, routed_scaling_factor=1.0, eps=1e-20)
    ex, ri, counts, _ = npu.npu_moe_init_routing_v2(L.x, idx, active_num=L.T * L.K, expert_num=L.E,
                                                    expert_tokens_num_type=1, expert_tokens_num_flag=True,
                                                    row_idx_type=0)
    q, s = npu.npu_dynamic_quant(ex)
    return y, idx, ex, ri, counts, q, s


def _ranges(counts):
    ends = torch.cumsum(counts, 0).tolist()
    return [(e, 0 if e == 0 else ends[e - 1], ends[e]) for e in range(len(ends)) if ends[e] > (0 if e == 0 else ends[e - 1])]


def test_cfg4_routing_and_quant_as_benched(layer):
    L = layer
    y, idx, ex, ri, counts, q, s = _stages(L)
    wy, widx, _ = G.moe_gating_top_k(L.logits.cpu().numpy(), L.K, L.bias.cpu().numpy(), 4, 8, 1, 0, 1, False, 1.0,
                                     1e-20)
    np.testing.assert_array_equal(idx.cpu().numpy(), widx)
    np.testing.assert_allclose(y.cpu().numpy(), wy, rtol=1e-6, atol=1e-7)
    # the permutation does not depend on x: route 8 columns through the oracle
    _, wri, wcounts, _ = G.moe_init_routing_v2(np.zeros((L.T, 8), np.float32), widx, None, L.T * L.K, 0, L.E, 1, 0)
    np.testing.assert_array_equal(ri.cpu().numpy(), wri)
    np.testing.assert_array_equal(counts.cpu().numpy(), wcounts)
    c = counts.cpu()
    assert int(c.max()) > 6 * 128, "the benched routing should give some expert >= 7 row tiles of 128"
    # expanded rows: row i holds token sorted_slot(i) // k (the gather form of row_idx_type 0 is inverted)
    inv = torch.empty_like(ri)
    inv[ri.long()] = torch.arange(ri.numel(), device=DEV, dtype=ri.dtype)
    assert torch.equal(ex, L.x[(inv.long() // L.K)])
    # every quantised row against the oracle
    wq, ws = G.dynamic_quant(ex.float().cpu().numpy())
    assert_int8_close(q.cpu().numpy(), wq)
    np.testing.assert_allclose(s.cpu().numpy(), ws, rtol=1e-6)


def test_cfg4_gate_up_exact_for_every_live_expert(layer):
    L = layer
    _, _, _, _, counts, q, _ = _stages(L)
    acc = torch.ops.npu.npu_grouped_matmul([q], [L.w_gu], group_list=counts, split_item=3, group_type=0,
                                           group_list_type=1, output_dtype=torch.int32)[0]
    live = _ranges(counts)
    assert len(live) == int((counts > 0).sum())
    for e, b0, b1 in live:
        ref = torch.matmul(q[b0:b1].double(), L.w_gu[e].double()).round().long()
        assert torch.equal(acc[b0:b1].long(), ref), f"expert {e} rows [{b0}, {b1})"


def test_cfg4_dsq_and_down_projection_full_shape(layer):
    L = layer
    npu = torch.ops.npu
    _, _, _, _, counts, q, s = _stages(L)
    acc = npu.npu_grouped_matmul([q], [L.w_gu], group_list=counts, split_item=3, group_type=0, group_list_type=1,
                                 output_dtype=torch.int32)[0]
    q2, s2 = npu.npu_dequant_swiglu_quant(acc, weight_scale=L.s_gu, activation_scale=s, group_index=counts,
                                          activate_left=True, quant_mode=1)
    # the oracle on every row, group by group
    sgu = L.s_gu.cpu().numpy()
    acc_h, s_h, q2_h, s2_h = acc.cpu().numpy(), s.cpu().numpy(), q2.cpu().numpy(), s2.cpu().numpy()
    for e, b0, b1 in _ranges(counts):
        wq2, ws2 = G.dequant_swiglu_quant(acc_h[b0:b1], sgu[e], s_h[b0:b1], activate_left=True)
        assert_int8_close(q2_h[b0:b1], wq2)
        np.testing.assert_allclose(s2_h[b0:b1], ws2, rtol=1e-5, err_msg=f"group {e}")
    del acc_h
    del acc
    out = npu.npu_grouped_matmul([q2], [L.w_d], scale=[L.s_d], per_token_scale=[s2], group_list=counts,
                                 split_item=3, group_type=0, group_list_type=1, output_dtype=torch.bfloat16)[0]
    assert out.shape == (L.T * L.K, L.H) and out.dtype == torch.bfloat16
    for e, b0, b1 in _ranges(counts):
        ref = torch.matmul(q2[b0:b1].double(), L.w_d[e].double()) * L.s_d[e].double()[None, :] * \
            s2[b0:b1].double()[:, None]
        torch.testing.assert_close(out[b0:b1].float(), ref.float(), rtol=1e-2, atol=1e-2,
                                   msg=lambda m: f"expert {e}: {m}")


def test_cfg4_finalize_and_layer_graph_replay(layer):
    L = layer
    npu = torch.ops.npu
    y, idx, _, ri, counts, q, s = _stages(L)
    out = L.step()
    # finalize against the oracle for every token: each token's k expanded rows
    acc = npu.npu_grouped_matmul([q], [L.w_gu], group_list=counts, split_item=3, group_type=0, group_list_type=1,
                                 output_dtype=torch.int32)[0]
    q2, s2 = npu.npu_dequant_swiglu_quant(acc, weight_scale=L.s_gu, activation_scale=s, group_index=counts,
                                          activate_left=True, quant_mode=1)
    down = npu.npu_grouped_matmul([q2], [L.w_d], scale=[L.s_d], per_token_scale=[s2], group_list=counts,
                                  split_item=3, group_type=0, group_list_type=1, output_dtype=torch.bfloat16)[0]
    toks = torch.arange(0, L.T)
    rows = ri.view(L.T, L.K)[toks.to(DEV)].long()
    sub = down[rows.reshape(-1)].float().cpu().numpy()
    want = G.moe_finalize_routing(sub, None, None, None, y[toks.to(DEV)].cpu().numpy(),
                                  np.arange(sub.shape[0]), idx[toks.to(DEV)].cpu().numpy(), 2, "bf16")
    assert_close(out[toks.to(DEV)].float().cpu().numpy(), want)
    # the bench's hipGraph variant replays the same layer: equal to eager on each replay
    from torchair_amd.graph import HipGraphRunner
    runner = HipGraphRunner(lambda logits: L.step(), clone_input=False)
    for i in range(3):
        got = runner(L.logits).clone()
        assert torch.equal(got, out), f"replay {i}"
        torch.cuda.synchronize()
