"""Eager entry points of the fused ops (the ``torch_npu.npu_*`` / ``torchair.ops`` surface)."""
import torch

from . import _ops_impl  # noqa: F401


def npu_fused_infer_attention_score(*args, **kwargs):
    """torchair.ops.npu_fused_infer_attention_score (python/torchair/ops/__init__.py:5-7; tensor sequence
    lengths), the air:: op. The reference's eager impl of that op raises outside its max-autotune graph
    mode (_npu_fused_infer_attention_score.py:36-42); here the kernels run in every mode."""
    return torch.ops.air.npu_fused_infer_attention_score(*args, **kwargs)


def npu_fused_infer_attention_score_v2(*args, **kwargs):
    """torchair.ops.npu_fused_infer_attention_score_v2 (python/torchair/ops/__init__.py:10-12), the air::
    v2 op (tensor sequence lengths)."""
    return torch.ops.air.npu_fused_infer_attention_score_v2(*args, **kwargs)


npu_dynamic_quant = torch.ops.npu.npu_dynamic_quant
npu_dequant_swiglu_quant = torch.ops.npu.npu_dequant_swiglu_quant
npu_quant_matmul = torch.ops.npu.npu_quant_matmul
npu_grouped_matmul = torch.ops.npu.npu_grouped_matmul
npu_moe_gating_top_k = torch.ops.npu.npu_moe_gating_top_k
npu_moe_init_routing = torch.ops.npu.npu_moe_init_routing
npu_moe_init_routing_v2 = torch.ops.npu.npu_moe_init_routing_v2
npu_moe_finalize_routing = torch.ops.npu.npu_moe_finalize_routing
npu_add_rms_norm = torch.ops.npu.npu_add_rms_norm
npu_add_rms_norm_dynamic_quant = torch.ops.npu.npu_add_rms_norm_dynamic_quant
npu_scatter_pa_kv_cache = torch.ops.npu.npu_scatter_pa_kv_cache
npu_kv_rmsnorm_rope_cache = torch.ops.npu.npu_kv_rmsnorm_rope_cache
npu_kv_rmsnorm_rope_cache_v2 = torch.ops.npu.npu_kv_rmsnorm_rope_cache_v2
npu_grouped_matmul_swiglu_quant_v2 = torch.ops.npu.npu_grouped_matmul_swiglu_quant_v2
npu_grouped_matmul_finalize_routing = torch.ops.npu.npu_grouped_matmul_finalize_routing
npu_dynamic_quant_asymmetric = torch.ops.npu.npu_dynamic_quant_asymmetric
npu_swiglu = torch.ops.npu.npu_swiglu
npu_moe_compute_expert_tokens = torch.ops.npu.npu_moe_compute_expert_tokens
npu_scatter_pa_kv_cache_functional = torch.ops.npu.npu_scatter_pa_kv_cache_functional
