"""The golden fixtures in tests/golden/: the oracle must reproduce them bit for bit (CPU), and
the GPU kernels must match them to the parity bar (int outputs exact or +-1 LSB, floats 1e-2)."""
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import golden as G
from tests.golden import make_fixtures as MF
from tests.helpers import assert_close, assert_int8_close

HERE = Path(__file__).resolve().parent / "golden"
DEV = "cuda"


def _load(name):
    with np.load(HERE / f"{name}.npz") as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", sorted(MF.CASES))
def test_oracle_reproduces_fixture(name):
    want = _load(name)
    got = {k: np.asarray(v) for k, v in MF.CASES[name]().items()}
    assert set(got) == set(want)
    for k in want:
        assert got[k].dtype == want[k].dtype and got[k].shape == want[k].shape, k
        np.testing.assert_array_equal(got[k], want[k], err_msg=f"{name}.{k}")


def _bf(bits):
    return torch.from_numpy(bits.astype(np.uint16).view(np.int16)).view(torch.bfloat16).to(DEV)


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _np(t):
    return t.float().cpu().numpy() if t.dtype in (torch.bfloat16, torch.float16) else t.cpu().numpy()


@pytest.mark.gpu
def test_gpu_dynamic_quant_fixture():
    f = _load("dynamic_quant")
    y, s = torch.ops.npu.npu_dynamic_quant(_bf(f["x"]), dst_type=1)  # ScalarType code of int8
    assert_int8_close(_np(y), f["y"])
    np.testing.assert_allclose(_np(s), f["scale"], rtol=1e-6)
    y, s = torch.ops.npu.npu_dynamic_quant(_bf(f["x"]), smooth_scales=_t(f["smooth"]))
    assert_int8_close(_np(y), f["y_smooth"])
    np.testing.assert_allclose(_np(s), f["scale_smooth"], rtol=1e-6)


@pytest.mark.gpu
@pytest.mark.parametrize("left", [True, False])
def test_gpu_dequant_swiglu_quant_fixture(left):
    f = _load("dequant_swiglu_quant")
    y, s = torch.ops.npu.npu_dequant_swiglu_quant(_t(f["x"]), weight_scale=_t(f["weight_scale"]),
                                                  activation_scale=_t(f["activation_scale"]), quant_mode=1,
                                                  activate_left=left)
    tag = "left" if left else "right"
    assert_int8_close(_np(y), f["y_" + tag])
    np.testing.assert_allclose(_np(s), f["scale_" + tag], rtol=1e-5)


@pytest.mark.gpu
def test_gpu_quant_matmul_fixture():
    f = _load("quant_matmul")
    # integer dtype codes, as the reference converters pass them (int32 = 3, bf16 = 15)
    acc = torch.ops.npu.npu_quant_matmul(_t(f["x1"]), _t(f["x2"]), torch.ones(1, device=DEV), output_dtype=3)
    assert acc.dtype == torch.int32
    np.testing.assert_array_equal(_np(acc), f["acc"])
    out = torch.ops.npu.npu_quant_matmul(_t(f["x1"]), _t(f["x2"]), _t(f["scale"]),
                                         pertoken_scale=_t(f["pertoken_scale"]), output_dtype=15)
    assert out.dtype == torch.bfloat16
    assert_close(_np(out), f["out_bf16"])


@pytest.mark.gpu
def test_gpu_grouped_matmul_fixture():
    f = _load("grouped_matmul")
    m = f["counts"].sum()
    acc = torch.ops.npu.npu_grouped_matmul([_t(f["x"])], [_t(f["w"])], group_list=_t(f["counts"]), split_item=3,
                                           group_type=0, group_list_type=1, output_dtype=torch.int32)[0]
    np.testing.assert_array_equal(_np(acc)[:m], f["acc"][:m])
    out = torch.ops.npu.npu_grouped_matmul([_t(f["x"])], [_t(f["w"])], scale=[_t(f["scale"])],
                                           per_token_scale=[_t(f["per_token_scale"])], group_list=_t(f["counts"]),
                                           split_item=3, group_type=0, group_list_type=1,
                                           output_dtype=torch.bfloat16)[0]
    assert_close(_np(out)[:m], f["out_bf16"][:m])


@pytest.mark.gpu
def test_gpu_moe_layer_fixture():
    f = _load("moe_layer")
    npu = torch.ops.npu
    y, idx, _ = npu.npu_moe_gating_top_k(_t(f["logits"]), 8, bias=_t(f["bias"]), k_group=4, group_count=8,
                                         group_select_mode=1, renorm=0, norm_type=1, routed_scaling_factor=1.0,
                                         eps=1e-20)
    np.testing.assert_array_equal(_np(idx), f["expert_idx"])
    np.testing.assert_allclose(_np(y), f["weights"], rtol=1e-6, atol=1e-7)
    t = f["x"].shape[0]
    ex, ri, counts, _ = npu.npu_moe_init_routing_v2(_bf(f["x"]), _t(f["expert_idx"]), active_num=t * 8,
                                                    expert_num=64, expert_tokens_num_type=1,
                                                    expert_tokens_num_flag=True, row_idx_type=0)
    np.testing.assert_array_equal(ex.view(torch.int16).cpu().numpy().view(np.uint16), f["expanded_x"])
    np.testing.assert_array_equal(_np(ri), f["expanded_row_idx"])
    np.testing.assert_array_equal(_np(counts), f["counts"])
    out = npu.npu_moe_finalize_routing(ex, None, None, None, _t(f["weights"]), ri, _t(f["expert_idx"]),
                                       drop_pad_mode=2)
    assert_close(_np(out), G.bf16_bits_to_f32(f["finalized"]))


@pytest.mark.gpu
def test_gpu_paged_decode_fixture():
    f = _load("paged_decode")
    b, hq, d = f["q"].shape
    nblk, bs, hkv, _ = f["k_cache"].shape
    out, lse = torch.ops.air.npu_fused_infer_attention_score(
        _bf(f["q"]).reshape(b, 1, hq * d), _bf(f["k_cache"]).reshape(nblk, bs, hkv * d),
        _bf(f["v_cache"]).reshape(nblk, bs, hkv * d), actual_seq_lengths_kv=_t(f["lens"]),
        block_table=_t(f["block_table"]), num_heads=hq, num_key_value_heads=hkv, input_layout="BSH",
        block_size=bs, scale=1.0 / math.sqrt(d), softmax_lse_flag=True)
    assert_close(_np(out).reshape(b, hq, d), f["out"])
    got = _np(lse).reshape(b, hq)
    want = f["lse"].reshape(b, hq)
    np.testing.assert_array_equal(np.isfinite(got), np.isfinite(want))
    np.testing.assert_allclose(got[np.isfinite(want)], want[np.isfinite(want)], rtol=1e-3, atol=1e-3)


@pytest.mark.gpu
def test_gpu_prefill_fixture():
    f = _load("prefill")
    b, s, hq, d = f["q"].shape
    hkv = f["k"].shape[2]
    out, lse = torch.ops.air.npu_fused_infer_attention_score(
        _bf(f["q"]).reshape(b, s, hq * d), _bf(f["k"]).reshape(b, s, hkv * d), _bf(f["v"]).reshape(b, s, hkv * d),
        actual_seq_lengths=_t(f["lq"]), actual_seq_lengths_kv=_t(f["lkv"]), num_heads=hq, num_key_value_heads=hkv,
        input_layout="BSH", scale=1.0 / math.sqrt(d), sparse_mode=3, softmax_lse_flag=True)
    assert_close(_np(out).reshape(b, s, hq, d), f["out"])
    got = _np(lse).reshape(f["lse"].shape)
    fin = np.isfinite(f["lse"])
    np.testing.assert_array_equal(np.isfinite(got), fin)
    np.testing.assert_allclose(got[fin], f["lse"][fin], rtol=1e-3, atol=1e-3)


@pytest.mark.gpu
def test_gpu_add_rms_norm_dynamic_quant_fixture():
    f = _load("add_rms_norm_dynamic_quant")
    y1, y2, x, s1, s2 = torch.ops.npu.npu_add_rms_norm_dynamic_quant(
        _bf(f["x1"]), _bf(f["x2"]), _bf(f["gamma"]), smooth_scale1=_t(f["smooth"]), output_mask=[True, False])
    assert_int8_close(_np(y1), f["q_y"])
    np.testing.assert_allclose(_np(s1), f["q_scale"], rtol=1e-5)
    np.testing.assert_array_equal(x.view(torch.int16).cpu().numpy().view(np.uint16), f["x_out"])
    y, rstd, xo = torch.ops.npu.npu_add_rms_norm(_bf(f["x1"]), _bf(f["x2"]), _bf(f["gamma"]))
    got = y.view(torch.int16).cpu().numpy().view(np.uint16)
    np.testing.assert_array_equal(got, f["y"])
    np.testing.assert_allclose(_np(rstd), f["rstd"], rtol=1e-6)
