"""Converters for the fused ops on the hot path.

Each mirrors the reference converter of the same op (file:line below) but lowers the FX
node onto the ``torch.library`` op served by libtai_kernels.so instead of a GE node, so the
lowered graph calls the HIP kernels directly and can be captured into a hipGraph.
"""
from __future__ import annotations

import torch

from . import _ops_impl  # noqa: F401  (defines the ops)
from .converter import Support, declare_supported, register_fx_node_ge_converter

npu = torch.ops.npu
air = torch.ops.air
npu_inference = torch.ops.npu_inference


def _identity(op):
    def convert(*args, meta_outputs=None, **kwargs):
        return op(*args, **kwargs)
    convert.__name__ = f"convert_{op}"
    return convert


# python/torchair/_ge_concrete_graph/ge_converter/custom/npu_dynamic_quant.py:4-8
declare_supported([
    Support(torch.empty(64, 16384, dtype=torch.float16)),
    Support(torch.empty(64, 16384, dtype=torch.bfloat16)),
])(register_fx_node_ge_converter(npu.npu_dynamic_quant.default)(_identity(npu.npu_dynamic_quant.default)))
# .../custom/npu_dynamic_quant.py:44-48 (declared cases as for npu_dynamic_quant)
declare_supported([
    Support(torch.empty(64, 16384, dtype=torch.float16)),
    Support(torch.empty(64, 16384, dtype=torch.bfloat16)),
])(register_fx_node_ge_converter(npu.npu_dynamic_quant_asymmetric.default)(
    _identity(npu.npu_dynamic_quant_asymmetric.default)))
# .../custom/npu_dequant_swiglu_quant.py:5
register_fx_node_ge_converter(npu.npu_dequant_swiglu_quant.default)(_identity(npu.npu_dequant_swiglu_quant.default))
register_fx_node_ge_converter(npu_inference.npu_dequant_swiglu_quant.default)(
    _identity(npu_inference.npu_dequant_swiglu_quant.default))
# .../custom/quantmatmul.py:63
register_fx_node_ge_converter(npu.npu_quant_matmul.default)(_identity(npu.npu_quant_matmul.default))
# .../custom/grouped_matmul.py:364-365
register_fx_node_ge_converter(npu.npu_grouped_matmul.default)(_identity(npu.npu_grouped_matmul.default))
register_fx_node_ge_converter(npu.npu_grouped_matmul.List)(_identity(npu.npu_grouped_matmul.List))
# .../custom/npu_moe_gating_top_k.py:4
register_fx_node_ge_converter(npu.npu_moe_gating_top_k.default)(_identity(npu.npu_moe_gating_top_k.default))
register_fx_node_ge_converter(npu_inference.npu_moe_gating_top_k.default)(
    _identity(npu_inference.npu_moe_gating_top_k.default))
# .../custom/moe_init_routing.py:4-10
declare_supported([
    Support(torch.empty(3, 4), torch.tensor([[0, 3], [1, 4], [2, 5]], dtype=torch.int32),
            torch.tensor([[1, 0], [2, 1], [0, 2]], dtype=torch.int32), active_num=3),
])(register_fx_node_ge_converter(npu.npu_moe_init_routing.default)(_identity(npu.npu_moe_init_routing.default)))
# .../custom/npu_moe_init_routing_v2.py:41
register_fx_node_ge_converter(npu.npu_moe_init_routing_v2.default)(_identity(npu.npu_moe_init_routing_v2.default))
# .../custom/npu_moe_finalize_routing.py:4-21 (the declared cases: 12 tokens, k = 2, 3 experts, hidden 7)
def _fin_cases():
    rows = torch.arange(24, dtype=torch.int32)
    experts = torch.tensor([[0, 1], [2, 0], [1, 1], [2, 2], [0, 2], [1, 0], [0, 0], [2, 1], [1, 2], [0, 1],
                            [2, 0], [1, 2]], dtype=torch.int32)
    f16, f32 = torch.float16, torch.float32
    e = torch.empty
    return [
        Support(e(24, 7, dtype=f16), e(12, 7, dtype=f16), e(12, 7, dtype=f16), e(3, 7, dtype=f16), e(12, 2, dtype=f16),
                rows, experts),
        Support(e(24, 7, dtype=f16), e(12, 7, dtype=f16), None, e(3, 7, dtype=f16), e(12, 2, dtype=f16), rows, experts),
        Support(e(24, 7, dtype=f32), e(12, 7, dtype=f32), None, e(3, 7, dtype=f32), e(12, 2, dtype=f32), rows, experts),
        Support(e(24, 7, dtype=f32), None, None, e(3, 7, dtype=f32), e(12, 2, dtype=f32), rows, experts),
        Support(e(24, 7, dtype=f32), None, None, None, e(12, 2, dtype=f32), rows, experts),
    ]


declare_supported(_fin_cases())(
    register_fx_node_ge_converter(npu.npu_moe_finalize_routing.default)(_identity(npu.npu_moe_finalize_routing.default)))
# .../custom/fused_infer_attention_score.py:4 and python/torchair/ops/_npu_fused_infer_attention_score.py:46-58
register_fx_node_ge_converter(npu.npu_fused_infer_attention_score.default)(
    _identity(npu.npu_fused_infer_attention_score.default))
register_fx_node_ge_converter(air.npu_fused_infer_attention_score.default)(
    _identity(air.npu_fused_infer_attention_score.default))
# python/torchair/ops/_npu_fused_infer_attention_score_v2.py:48-62 (its declared cases) and
# .../custom/fused_infer_attention_score_v2.py:14
declare_supported([
    Support(torch.empty(1, 2048, 40 * 128, dtype=torch.float16), torch.empty(1, 2048, 40 * 128, dtype=torch.float16),
            torch.empty(1, 2048, 40 * 128, dtype=torch.float16), num_query_heads=40, input_layout="BSH"),
    Support(torch.empty(1, 40, 2048, 128, dtype=torch.float16), torch.empty(1, 40, 2048, 128, dtype=torch.float16),
            torch.empty(1, 40, 2048, 128, dtype=torch.float16), num_query_heads=40, input_layout="BNSD"),
    Support(torch.empty(1, 40, 2048, 128, dtype=torch.float16), torch.empty(1, 40, 2048, 128, dtype=torch.float16),
            torch.empty(1, 40, 2048, 128, dtype=torch.float16), input_layout="BNSD", num_query_heads=40,
            softmax_scale=0.0884),
])(register_fx_node_ge_converter(air.npu_fused_infer_attention_score_v2.default)(
    _identity(air.npu_fused_infer_attention_score_v2.default)))
register_fx_node_ge_converter(npu.npu_fused_infer_attention_score_v2.default)(
    _identity(npu.npu_fused_infer_attention_score_v2.default))
# .../custom/npu_add_rms_norm.py:4-13, npu_add_rms_norm_dynamic_quant.py:8-21
register_fx_node_ge_converter(npu.npu_add_rms_norm.default)(_identity(npu.npu_add_rms_norm.default))
# .../custom/npu_add_rms_norm_dynamic_quant.py:4-7
declare_supported([
    Support(torch.empty(1, 2, 3, dtype=torch.float16), torch.empty(1, 2, 3, dtype=torch.float16),
            torch.empty(3, dtype=torch.float16), output_mask=[True, True]),
    Support(torch.empty(1, 2, 3, dtype=torch.float16), torch.empty(1, 2, 3, dtype=torch.float16),
            torch.empty(3, dtype=torch.float16), smooth_scale1=torch.empty(3, dtype=torch.float16),
            output_mask=[True, True]),
])(register_fx_node_ge_converter(npu.npu_add_rms_norm_dynamic_quant.default)(
    _identity(npu.npu_add_rms_norm_dynamic_quant.default)))
# .../custom/npu_scatter_pa_kv_cache.py:44-74
register_fx_node_ge_converter(npu.npu_scatter_pa_kv_cache_functional.default)(
    _identity(npu.npu_scatter_pa_kv_cache_functional.default))
# .../custom/npu_kv_rmsnorm_rope_cache.py:4-66 and python/torchair/_contrib/custom_torch_ops/npu_kv_rmsnorm_rope_cache.py:17
register_fx_node_ge_converter(npu.npu_kv_rmsnorm_rope_cache.default)(_identity(npu.npu_kv_rmsnorm_rope_cache.default))
register_fx_node_ge_converter(npu.npu_kv_rmsnorm_rope_cache_v2_functional.default)(
    _identity(npu.npu_kv_rmsnorm_rope_cache_v2_functional.default))
register_fx_node_ge_converter(npu_inference.npu_kv_rmsnorm_rope_cache.default)(
    _identity(npu_inference.npu_kv_rmsnorm_rope_cache.default))
# .../custom/grouped_matmul_swiglu_quant_v2.py:86-166, grouped_matmul_finalize_routing.py:32-133
register_fx_node_ge_converter(npu.npu_grouped_matmul_swiglu_quant_v2.default)(
    _identity(npu.npu_grouped_matmul_swiglu_quant_v2.default))
register_fx_node_ge_converter(npu.npu_grouped_matmul_finalize_routing.default)(
    _identity(npu.npu_grouped_matmul_finalize_routing.default))

# .../custom/npu_swiglu.py:4-14 (its declared cases)
declare_supported([
    Support(torch.empty(2, 2, dtype=torch.float32)),
    Support(torch.empty(2, 2, dtype=torch.float16)),
])(register_fx_node_ge_converter(npu.npu_swiglu.default)(_identity(npu.npu_swiglu.default)))
# .../custom/npu_moe_compute_expert_tokens.py:4-11
register_fx_node_ge_converter(npu.npu_moe_compute_expert_tokens.default)(
    _identity(npu.npu_moe_compute_expert_tokens.default))
