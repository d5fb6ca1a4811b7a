"""CPU ("debug path") kernels of the npu fused ops, backed by the oracle - TEST INFRASTRUCTURE ONLY.

``register()`` installs the oracle as the CPU implementation of the torch.library ops, so that
``torch.compile(backend=get_npu_backend())`` can run a model on CPU tensors. Used by tests and
by bench.py's cpu_baseline leg; the product never imports it.
"""
from __future__ import annotations

import numpy as np
import torch

from . import golden as G

_DONE = False
_NAMES = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}


def _np(t):
    if t is None:
        return None
    if t.dtype in (torch.bfloat16, torch.float16):
        t = t.float()
    return t.detach().cpu().numpy()


def _t(a, dtype=None):
    out = torch.from_numpy(np.ascontiguousarray(a))
    return out.to(dtype) if dtype is not None else out


def _code(v):
    from torchair_amd._ops_impl import scalar_type_code
    return scalar_type_code(v)


def register() -> None:
    global _DONE
    if _DONE:
        return
    import torchair_amd  # noqa: F401  (defines the ops)
    from torchair_amd._ops_impl import LIBS, dtype_of_code

    def dq(input, *, smooth_scales=None, group_index=None, dst_type=None, quant_mode="pertoken", dst_type_max=0.0):
        if quant_mode == "pertensor" or (dst_type_max or 0.0) != 0.0:
            y, s, _ = G.dynamic_quant_v2(_np(input), _np(smooth_scales), _np(group_index), True,
                                         quant_mode == "pertensor", dst_type_max or 0.0)
            return _t(y), _t(s)
        y, s = G.dynamic_quant(_np(input), _np(smooth_scales), _np(group_index))
        return _t(y), _t(s)

    def dq_asym(input, *, smooth_scales=None, group_index=None, dst_type=None, quant_mode="pertoken",
                dst_type_max=0.0):
        y, s, o = G.dynamic_quant_v2(_np(input), _np(smooth_scales), _np(group_index), False,
                                     quant_mode == "pertensor", 0.0)
        return _t(y), _t(s), _t(o)

    def dsq(x, *, weight_scale=None, activation_scale=None, bias=None, quant_scale=None, quant_offset=None,
            group_index=None, activate_left=False, quant_mode=0, dst_type=None, round_mode=None, activate_dim=None,
            swiglu_mode=0, clamp_limit=7.0, glu_alpha=1.702, glu_bias=1.0):
        b = None if bias is None else (bias.numpy() if bias.dtype == torch.int32 else _np(bias))
        y, s = G.dequant_swiglu_quant(x.numpy(), _np(weight_scale), _np(activation_scale), b, _np(quant_scale),
                                      _np(group_index), activate_left, quant_mode, _np(quant_offset))
        return _t(y), _t(s)

    def qmm(x1, x2, scale, *, offset=None, pertoken_scale=None, bias=None, output_dtype=None, x1_dtype=None,
            x2_dtype=None, pertoken_scale_dtype=None, scale_dtype=None, group_sizes=None):
        code = _code(output_dtype)
        od = torch.int8 if code is None else dtype_of_code(code)
        name = {torch.int32: "int32", torch.int8: "int8"}.get(od) or _NAMES[od]
        b = None if bias is None else (bias.numpy() if bias.dtype == torch.int32 else _np(bias))
        k = x1.shape[-1]
        out = G.quant_matmul(x1.reshape(-1, k).numpy(), x2.numpy(), _np(scale).reshape(-1) if scale is not None
                             else None, _np(pertoken_scale), b, name,
                             offset=None if offset is None else _np(offset).reshape(-1))
        return _t(out, od).reshape(list(x1.shape[:-1]) + [x2.shape[-1]])

    def gmm(x, weight, *, bias=None, scale=None, offset=None, antiquant_scale=None, antiquant_offset=None,
            per_token_scale=None, group_list=None, activation_input=None, activation_quant_scale=None,
            activation_quant_offset=None, split_item=0, group_type=None, group_list_type=0, act_type=0,
            tuning_config=None, output_dtype=None):
        od = dtype_of_code(_code(output_dtype))
        name = "int32" if od == torch.int32 else _NAMES[od]
        w = weight[0] if len(weight) == 1 else torch.stack(list(weight))
        gl = group_list.numpy() if isinstance(group_list, torch.Tensor) else np.asarray(group_list)
        b = None
        if bias:
            b = bias[0].numpy() if bias[0].dtype == torch.int32 else _np(bias[0])
        out = G.grouped_matmul(x[0].numpy(), w.numpy(), gl, group_list_type, _np(scale[0]) if scale else None,
                               _np(per_token_scale[0]) if per_token_scale else None, b, name)
        return [_t(out, od)]

    def gate(x, k, *, bias=None, k_group=1, group_count=1, group_select_mode=0, renorm=0, norm_type=0,
             out_flag=False, routed_scaling_factor=1.0, eps=1e-20):
        y, idx, out = G.moe_gating_top_k(_np(x), k, _np(bias), k_group, group_count, group_select_mode, renorm,
                                         norm_type, out_flag, routed_scaling_factor, eps, _NAMES[x.dtype])
        return _t(y, x.dtype), _t(idx), _t(out)

    def init_v2(x, expert_idx, *, scale=None, offset=None, active_num=-1, expert_capacity=-1, expert_num=-1,
                drop_pad_mode=0, expert_tokens_num_type=0, expert_tokens_num_flag=False, quant_mode=-1,
                active_expert_range=(), row_idx_type=0):
        t, k = expert_idx.shape
        n = t * k
        rows = n if (active_num is None or active_num <= 0 or active_num >= n) else active_num
        lo, hi = (active_expert_range[0], active_expert_range[1]) if active_expert_range else (0, expert_num)
        if quant_mode == 1:  # dynamic quant of every expanded row (no smooth scale)
            ex, ri, tok, _ = G.moe_init_routing_v2(_np(x), expert_idx.numpy(), None, rows, lo, hi,
                                                   expert_tokens_num_type, row_idx_type)
            q, s = G.dynamic_quant(ex)
            return _t(q), _t(ri), _t(tok), _t(s)
        ex, ri, tok, es = G.moe_init_routing_v2(_np(x), expert_idx.numpy(), _np(scale), rows, lo, hi,
                                                expert_tokens_num_type, row_idx_type)
        es_t = _t(es) if es is not None else torch.empty(0, dtype=torch.float32)
        return _t(ex, x.dtype), _t(ri), _t(tok), es_t

    def init_v2_rows(x, expert_idx, *, active_num=-1, expert_num=-1, expert_tokens_num_type=0,
                     active_expert_range=(), row_idx_type=0):
        # tai::moe_init_routing_v2_rows: the routing of the quantised token rows, with the token row
        # of every expanded row in place of the rows themselves
        t, k = expert_idx.shape
        n = t * k
        rows = n if (active_num is None or active_num <= 0 or active_num >= n) else active_num
        lo, hi = (active_expert_range[0], active_expert_range[1]) if active_expert_range else (0, expert_num)
        q, s = G.dynamic_quant(_np(x))
        _, ri, tok, es = G.moe_init_routing_v2(q, expert_idx.numpy(), s, rows, lo, hi, expert_tokens_num_type,
                                               row_idx_type)
        a_rows = np.zeros(rows, np.int32)
        ri = np.asarray(ri)
        if row_idx_type == 0:
            for p_, d in enumerate(ri):
                if 0 <= d < rows:
                    a_rows[d] = p_ // k
        else:
            for d in range(min(rows, len(ri))):
                if ri[d] >= 0:
                    a_rows[d] = ri[d] // k
        return _t(q), _t(a_rows), _t(ri), _t(tok), _t(es)

    def gmm_gather(x, a_rows, weight, group_list, *, scale=None, per_token_scale=None, bias=None,
                   group_list_type=0, output_dtype=None):
        xs = [x[a_rows.long()]]
        return gmm(xs, [weight], bias=None if bias is None else [bias], scale=None if scale is None else [scale],
                   per_token_scale=None if per_token_scale is None else [per_token_scale], group_list=group_list,
                   split_item=3, group_type=0, group_list_type=group_list_type, output_dtype=output_dtype)[0]

    def gsq_gather(x, a_rows, weight, weight_scale, x_scale, group_list, *, group_list_type=0):
        return gsq(x[a_rows.long()], [weight], [weight_scale], x_scale, group_list, group_list_type=group_list_type)

    def fia_v2(query, key, value, *, pse_shift=None, atten_mask=None, actual_seq_qlen=None, actual_seq_kvlen=None,
               block_table=None, num_query_heads=1, num_key_value_heads=0, softmax_scale=1.0, pre_tokens=2147483647,
               next_tokens=2147483647, input_layout="BSH", sparse_mode=0, return_softmax_lse=False, **unused):
        # dense prefill of npu_fused_infer_attention_score_v2 (BSH / BSND / BNSD, no mask or a causal
        # sparse_mode 2 / 3): prefill_attention over [B, S, N, D] views
        assert block_table is None and pse_shift is None and atten_mask is None
        assert all(v in (None, 0, False) for v in unused.values()), "only the dense prefill cases are served"
        hq = num_query_heads
        hkv = num_key_value_heads or hq

        def bsnd(t, n):
            if input_layout == "BSH":
                return t.reshape(t.shape[0], t.shape[1], n, -1)
            return t.permute(0, 2, 1, 3) if input_layout == "BNSD" else t
        q, k, v = bsnd(query, hq), bsnd(key, hkv), bsnd(value, hkv)
        causal = {0: 0, 2: 2, 3: 1}[sparse_mode]
        sq = None if actual_seq_qlen is None else np.asarray(actual_seq_qlen)
        skv = None if actual_seq_kvlen is None else np.asarray(actual_seq_kvlen)
        o, lse = G.prefill_attention(_np(q), _np(k), _np(v), sq, skv, causal, softmax_scale)
        out = _t(o, query.dtype)
        if input_layout == "BSH":
            out = out.reshape(query.shape[0], query.shape[1], -1)
        elif input_layout == "BNSD":
            out = out.permute(0, 2, 1, 3).contiguous()
        lse_t = _t(lse).unsqueeze(-1) if return_softmax_lse else torch.empty(0, dtype=torch.float32)
        return out, lse_t

    def swiglu(x, dim=-1):
        return _t(G.swiglu(_np(x), dim, _NAMES[x.dtype]), x.dtype)

    def cet(sorted_experts, num_experts):
        return _t(G.moe_compute_expert_tokens(sorted_experts.numpy(), num_experts))

    def init_legacy(x, row_idx, expert_idx, active_num):
        ex, ri, ei = G.moe_init_routing(_np(x), row_idx.numpy(), expert_idx.numpy(), active_num)
        return _t(ex, x.dtype), _t(ri), _t(ei)

    def finalize(expanded_permuted_rows, skip1, skip2, bias, scales, expanded_src_to_dst_row,
                 export_for_source_row, drop_pad_mode=0):
        ex = expanded_permuted_rows
        y = G.moe_finalize_routing(_np(ex), _np(skip1), _np(skip2), _np(bias), _np(scales),
                                   expanded_src_to_dst_row.numpy(),
                                   None if export_for_source_row is None else export_for_source_row.numpy(),
                                   0 if drop_pad_mode is None else drop_pad_mode, _NAMES[ex.dtype])
        return _t(y, ex.dtype)

    def arn(x1, x2, gamma, epsilon=1e-6):
        y, rstd, x = G.add_rms_norm(_np(x1), _np(x2), _np(gamma), epsilon, _NAMES[x1.dtype])
        return _t(y, x1.dtype), _t(rstd), _t(x, x1.dtype)

    def arnq(x1, x2, gamma, *, smooth_scale1=None, smooth_scale2=None, beta=None, epsilon=1e-6, output_mask=()):
        mask = list(output_mask or [])
        second = bool(mask[1]) if mask else smooth_scale2 is not None
        y1, y2, x, s1, s2 = G.add_rms_norm_dynamic_quant(_np(x1), _np(x2), _np(gamma), _np(smooth_scale1),
                                                         _np(smooth_scale2), _np(beta), epsilon, second,
                                                         _NAMES[x1.dtype])
        if not second:
            y2, s2 = np.zeros_like(y1), np.zeros_like(s1)
        return _t(y1), _t(y2), _t(x, x1.dtype), _t(s1), _t(s2)

    def _cache_np(c):
        return c.numpy() if c.dtype in (torch.int8, torch.int32, torch.int64, torch.float32) else _np(c)

    def scatter_functional(key, value, key_cache, value_cache, slot_mapping, *, compress_lens=None,
                           compress_seq_offsets=None, seq_lens=None, cache_mode="Norm"):
        kc, vc = G.scatter_pa_kv_cache(_cache_np(key), _cache_np(value), _cache_np(key_cache),
                                       _cache_np(value_cache), slot_mapping.numpy(), cache_mode)
        return _t(kc, key_cache.dtype), _t(vc, value_cache.dtype)

    def scatter_inplace(key, value, key_cache, value_cache, slot_mapping, *, compress_lens=None,
                        compress_seq_offsets=None, seq_lens=None, cache_mode="Norm"):
        kc, vc = scatter_functional(key, value, key_cache, value_cache, slot_mapping, cache_mode=cache_mode)
        key_cache.copy_(kc)
        value_cache.copy_(vc)

    def _kv(kv, gamma, cos, sin, index, k_cache, ckv_cache, k_rope_scale, c_kv_scale, k_rope_offset, c_kv_offset,
            epsilon, cache_mode):
        per_token = ckv_cache.dtype == torch.int8 and c_kv_scale is not None and c_kv_scale.dim() >= 2
        res = G.kv_rmsnorm_rope_cache(_np(kv), _np(gamma), _np(cos), _np(sin), index.numpy(), _cache_np(k_cache),
                                      _cache_np(ckv_cache), epsilon, cache_mode, _np(k_rope_scale),
                                      _np(k_rope_offset), None if per_token else _np(c_kv_scale), _np(c_kv_offset),
                                      c_kv_scale.numpy() if per_token else None, _NAMES[kv.dtype])
        kc, cc, kr, ckv = res[:4]
        return (_t(kc, k_cache.dtype), _t(cc, ckv_cache.dtype), _t(kr, kv.dtype), _t(ckv, kv.dtype),
                _t(res[4]) if per_token else None)

    def kv_v2(kv, gamma, cos, sin, index, k_cache, ckv_cache, *, k_rope_scale=None, c_kv_scale=None,
              k_rope_offset=None, c_kv_offset=None, v=None, epsilon=1e-5, cache_mode="Norm", is_output_kv=False):
        kc, cc, kr, ckv, ts = _kv(kv, gamma, cos, sin, index, k_cache, ckv_cache, k_rope_scale, c_kv_scale,
                                  k_rope_offset, c_kv_offset, epsilon, cache_mode)
        k_cache.copy_(kc)
        ckv_cache.copy_(cc)
        if ts is not None:
            c_kv_scale.copy_(ts)
        return kr, ckv

    def kv_v2f(kv, gamma, cos, sin, index, k_cache, ckv_cache, *, k_rope_scale=None, c_kv_scale=None,
               k_rope_offset=None, c_kv_offset=None, v=None, epsilon=1e-5, cache_mode="Norm", is_output_kv=False):
        kc, cc, kr, ckv, _ = _kv(kv, gamma, cos, sin, index, k_cache, ckv_cache, k_rope_scale, c_kv_scale,
                                 k_rope_offset, c_kv_offset, epsilon, cache_mode)
        return kr, ckv, kc, cc

    def kv_legacy(kv, gamma, cos, sin, index, k_cache, ckv_cache, *, k_rope_scale=None, c_kv_scale=None,
                  k_rope_offset=None, c_kv_offset=None, v=None, epsilon=1e-5, cache_mode="Norm", is_output_kv=False):
        kc, cc, kr, ckv, _ = _kv(kv, gamma, cos, sin, index, k_cache, ckv_cache, k_rope_scale, c_kv_scale,
                                 k_rope_offset, c_kv_offset, epsilon, cache_mode)
        return kc, cc, kr, ckv

    def gsq(x, weight, weight_scale, x_scale, group_list, *, smooth_scale=None, weight_assist_matrix=None,
            bias=None, dequant_mode=0, dequant_dtype=0, quant_mode=0, quant_dtype=1, group_list_type=0,
            tuning_config=None, x_dtype=None, weight_dtype=None, weight_scale_dtype=None, x_scale_dtype=None):
        y, s = G.grouped_matmul_swiglu_quant(x.numpy(), weight[0].numpy(), _np(weight_scale[0]), _np(x_scale),
                                             group_list.numpy(), group_list_type)
        return _t(y), _t(s)

    def gfr(x, w, group_list, *, scale=None, bias=None, offset=None, pertoken_scale=None, shared_input=None,
            logit=None, row_index=None, dtype=None, shared_input_weight=1.0, shared_input_offset=0, output_bs=0,
            group_list_type=1, tuning_config=()):
        y = G.grouped_matmul_finalize_routing(x.numpy(), w.numpy(), group_list.numpy(),
                                              1 if group_list_type is None else group_list_type, _np(scale),
                                              _np(pertoken_scale), _np(bias), _np(logit),
                                              None if row_index is None else row_index.numpy(), _np(shared_input),
                                              1.0 if shared_input_weight is None else shared_input_weight,
                                              shared_input_offset or 0, output_bs or 0)
        return _t(y)

    for ns in ("npu",):
        lib = LIBS[ns]
        lib.impl("npu_grouped_matmul_swiglu_quant_v2", gsq, "CPU")
        lib.impl("npu_grouped_matmul_finalize_routing", gfr, "CPU")
        lib.impl("npu_add_rms_norm", arn, "CPU")
        lib.impl("npu_add_rms_norm_dynamic_quant", arnq, "CPU")
        lib.impl("npu_scatter_pa_kv_cache", scatter_inplace, "CPU")
        lib.impl("npu_scatter_pa_kv_cache_functional", scatter_functional, "CPU")
        lib.impl("npu_kv_rmsnorm_rope_cache_v2", kv_v2, "CPU")
        lib.impl("npu_kv_rmsnorm_rope_cache_v2_functional", kv_v2f, "CPU")
        lib.impl("npu_kv_rmsnorm_rope_cache", kv_legacy, "CPU")
        LIBS["npu_inference"].impl("npu_kv_rmsnorm_rope_cache", kv_legacy, "CPU")
        lib.impl("npu_dynamic_quant", dq, "CPU")
        lib.impl("npu_dynamic_quant_asymmetric", dq_asym, "CPU")
        lib.impl("npu_quant_matmul", qmm, "CPU")
        lib.impl("npu_grouped_matmul", gmm, "CPU")
        lib.impl("npu_moe_init_routing_v2", init_v2, "CPU")
        LIBS["tai"].impl("moe_init_routing_v2_rows", init_v2_rows, "CPU")
        LIBS["tai"].impl("grouped_matmul_gather", gmm_gather, "CPU")
        LIBS["tai"].impl("grouped_matmul_swiglu_quant_gather", gsq_gather, "CPU")
        LIBS["air"].impl("npu_fused_infer_attention_score_v2", fia_v2, "CPU")
        lib.impl("npu_moe_init_routing", init_legacy, "CPU")
        lib.impl("npu_swiglu", swiglu, "CPU")
        lib.impl("npu_moe_compute_expert_tokens", cet, "CPU")
        lib.impl("npu_moe_finalize_routing", finalize, "CPU")
    for ns in ("npu", "npu_inference"):
        LIBS[ns].impl("npu_dequant_swiglu_quant", dsq, "CPU")
        LIBS[ns].impl("npu_moe_gating_top_k", gate, "CPU")
    _DONE = True
