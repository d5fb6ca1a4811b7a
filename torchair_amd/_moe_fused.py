"""Private ops of the compiled graph's routing -> grouped GEMM fusion (libtai_kernels.so).

npu_moe_init_routing_v2 (dropless, quant_mode 1 without smooth scales) materialises expanded_x: every
routed slot's int8 token row, T * k rows (235 MB at DeepSeek-V3 decode shapes), which the gate_up
npu_grouped_matmul then reads back. When that GEMM is the rows' only consumer, the pattern pass
(patterns.fuse_routing_grouped_matmul) replaces the pair by

  tai::moe_init_routing_v2_rows  the same routing, returning the T quantised token rows, their
                                 scales and a_rows (the token row of each expanded row) instead of
                                 the expanded rows; the other outputs are unchanged;
  tai::grouped_matmul_gather     npu_grouped_matmul over rows gathered through a_rows.

Product row r of the GEMM equals expanded_x[r] @ w[e] exactly (the same int8 bytes are multiplied),
so the rewrite changes no value. Neither op has a counterpart in the reference's interface; both are
built from the reference ops' semantics (npu_moe_init_routing_v2.py:41-91, grouped_matmul.py:210-365).
"""
from __future__ import annotations

import torch

from . import _lib
from ._lib import DT_NONE, LAYOUT_KN, LAYOUT_NK
from ._ops_impl import (LIBS, _DT, _check, _f32, _gmm_out_dtype, _on_gpu, _p, _stream, _v2_expert_range)

LIBS["tai"] = torch.library.Library("tai", "FRAGMENT")


def _define(schema, fake, cuda):
    lib = LIBS["tai"]
    lib.define(schema)
    name = schema.split("(")[0]
    torch.library.register_fake(f"tai::{name}", fake, lib=lib)
    lib.impl(name, cuda, "CUDA")


# ============================================================================ routing without rows
def _rows_fake(x, expert_idx, *, active_num=-1, expert_num=-1, expert_tokens_num_type=0, active_expert_range=(),
               row_idx_type=0):
    t, k = expert_idx.shape
    n = t * k
    lo, hi = _v2_expert_range(expert_num, active_expert_range)
    rows = n if (active_num is None or active_num <= 0 or active_num >= n) else active_num
    return (x.new_empty((t, x.shape[1]), dtype=torch.int8), x.new_empty((rows,), dtype=torch.int32),
            x.new_empty((n,), dtype=torch.int32), x.new_empty((max(hi - lo, 0),), dtype=torch.int64),
            x.new_empty((rows,), dtype=torch.float32))


def _rows_cuda(x, expert_idx, *, active_num=-1, expert_num=-1, expert_tokens_num_type=0, active_expert_range=(),
               row_idx_type=0):
    """npu_moe_init_routing_v2(x, expert_idx, quant_mode=1, drop_pad_mode=0, ...) without expanded_x:
    returns (q [T, H] int8, a_rows [rows] int32, expanded_row_idx, expert_tokens, expanded_scale), where
    expanded_x would be q[a_rows] for the rows below the routed total (and zero past it)."""
    name = "tai::moe_init_routing_v2_rows"
    _on_gpu(x, expert_idx)
    _check(x.dim() == 2 and expert_idx.dim() == 2 and expert_idx.shape[0] == x.shape[0],
           f"{name}: x [T,H] and expert_idx [T,k]")
    _check(expert_idx.dtype == torch.int32, f"{name}: expert_idx must be int32")
    _check(expert_tokens_num_type in (0, 1), f"{name}: expert_tokens_num_type must be 0 or 1")
    lo, hi = _v2_expert_range(expert_num, active_expert_range)
    _check(hi > lo >= 0, f"{name}: expert_num or active_expert_range is required")
    q, s = torch.ops.npu.npu_dynamic_quant(x)
    _, a_rows, ri, tok, es = _rows_fake(x, expert_idx, active_num=active_num, expert_num=expert_num,
                                        active_expert_range=active_expert_range)
    t, k = expert_idx.shape
    if t == 0:
        return q, a_rows, ri, tok.zero_(), es
    ec = expert_idx.contiguous()
    ws_bytes = _lib.query("tai_moe_init_routing_workspace_size", t, k, hi - lo)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    _lib.call("tai_moe_init_routing_v2_rows", t, _p(ec), k, _p(s), a_rows.shape[0], lo, hi,
              int(expert_tokens_num_type), int(row_idx_type), _p(a_rows), _p(ri), _p(tok), _p(es), _p(ws), ws_bytes,
              _stream(ec))
    return q, a_rows, ri, tok, es


_define("moe_init_routing_v2_rows(Tensor x, Tensor expert_idx, *, int active_num=-1, int expert_num=-1, "
        "int expert_tokens_num_type=0, int[] active_expert_range=[], int row_idx_type=0) "
        "-> (Tensor, Tensor, Tensor, Tensor, Tensor)", _rows_fake, _rows_cuda)


# ============================================================================ grouped GEMM over gathered rows
def _gather_fake(x, a_rows, weight, group_list, *, scale=None, per_token_scale=None, bias=None, group_list_type=0,
                 output_dtype=None):
    return x.new_empty((a_rows.shape[0], weight.shape[-1]), dtype=_gmm_out_dtype([x], output_dtype))


def _gather_cuda(x, a_rows, weight, group_list, *, scale=None, per_token_scale=None, bias=None, group_list_type=0,
                 output_dtype=None):
    """npu_grouped_matmul([x[a_rows]], [weight], group_list=..., split_item 2/3, group_type 0) with the
    rows gathered by the kernel: out[r] = x[a_rows[r]] @ weight[group of r] and the same epilogue."""
    name = "tai::grouped_matmul_gather"
    _on_gpu(x, a_rows, weight, group_list, scale, per_token_scale, bias)
    _check(x.dtype == torch.int8 and x.dim() == 2, f"{name}: x must be int8 [T, K]")
    _check(a_rows.dtype == torch.int32 and a_rows.dim() == 1, f"{name}: a_rows must be int32 [M]")
    _check(weight.dtype == torch.int8 and weight.dim() == 3, f"{name}: weight must be int8 [E, K, N]")
    _check(group_list_type in (0, 1), f"{name}: group_list_type must be 0 (cumsum) or 1 (count)")
    e, k, n = weight.shape
    _check(x.shape[1] == k, f"{name}: x is [T, K] with the weight's K")
    out_dtype = _gmm_out_dtype([x], output_dtype)
    _check(out_dtype in (torch.int32, torch.bfloat16, torch.float16, torch.float32),
           f"{name}: output_dtype must be int32, bf16, fp16 or fp32")
    if weight.is_contiguous():
        wl, layout = weight, LAYOUT_KN
    elif weight.transpose(1, 2).is_contiguous():
        wl, layout = weight.transpose(1, 2), LAYOUT_NK
    else:
        wl, layout = weight.contiguous(), LAYOUT_KN
    gl = group_list.to(torch.int64).contiguous()
    _check(gl.numel() == e, f"{name}: group_list has {gl.numel()} entries, weight has {e} groups")
    sc = _f32(scale)
    if sc is not None:
        _check(sc.numel() == e * n, f"{name}: scale must be [E, N]")
    m = a_rows.shape[0]
    pts = _f32(per_token_scale)
    if pts is not None:
        _check(pts.numel() == m, f"{name}: per_token_scale must have M entries")
    bi, bias_dt = None, DT_NONE
    if bias is not None:
        bi = bias.contiguous() if bias.dtype == torch.int32 else _f32(bias)
        bias_dt = _DT[bi.dtype]
        _check(bi.numel() == e * n, f"{name}: bias must be [E, N]")
    _check(out_dtype == torch.int32 or sc is not None, f"{name}: floating output needs scale")
    out = torch.empty([m, n], dtype=out_dtype, device=x.device)
    if m > 0 and n > 0:
        xc, rc = x.contiguous(), a_rows.contiguous()
        ws_bytes = _lib.query("tai_grouped_matmul_workspace_size", m, n, e)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
        _lib.call("tai_grouped_matmul_gather", _p(xc), xc.shape[0], _p(rc), _p(wl), m, k, n, e, layout, _p(gl),
                  int(group_list_type), _p(sc), _p(pts), _p(bi), bias_dt, _DT[out_dtype], _p(out), _p(ws), ws_bytes,
                  _stream(xc))
    return out


_define("grouped_matmul_gather(Tensor x, Tensor a_rows, Tensor weight, Tensor group_list, *, Tensor? scale=None, "
        "Tensor? per_token_scale=None, Tensor? bias=None, int group_list_type=0, ScalarType? output_dtype=None) "
        "-> Tensor", _gather_fake, _gather_cuda)


# ============================================================================ gathered gate_up + SwiGLU quant
def _gsq_gather_fake(x, a_rows, weight, weight_scale, x_scale, group_list, *, group_list_type=0):
    m = a_rows.shape[0]
    return (x.new_empty((m, weight.shape[-1] // 2), dtype=torch.int8), x.new_empty((m,), dtype=torch.float32))


def _gsq_gather_cuda(x, a_rows, weight, weight_scale, x_scale, group_list, *, group_list_type=0):
    """npu_grouped_matmul_swiglu_quant_v2(x[a_rows], [weight], [weight_scale], x_scale, group_list) with the
    rows gathered by the kernel; the fold of tai::grouped_matmul_gather(int32) + npu_dequant_swiglu_quant."""
    from ._gmm_fused import _swiglu_packed
    from ._lib import LAYOUT_KN_SWIGLU
    name = "tai::grouped_matmul_swiglu_quant_gather"
    _on_gpu(x, a_rows, weight, weight_scale, x_scale, group_list)
    _check(x.dtype == torch.int8 and x.dim() == 2, f"{name}: x must be int8 [T, K]")
    _check(a_rows.dtype == torch.int32 and a_rows.dim() == 1, f"{name}: a_rows must be int32 [M]")
    _check(weight.dtype == torch.int8 and weight.dim() == 3, f"{name}: weight must be int8 [E, K, N]")
    _check(group_list_type in (0, 1), f"{name}: group_list_type must be 0 (cumsum) or 1 (count)")
    e, k, n = weight.shape
    _check(x.shape[1] == k and n % 2 == 0, f"{name}: x is [T, K] and the weight [E, K, N] with N even")
    if weight.is_contiguous():
        wl, layout = weight, LAYOUT_KN
        packed = _swiglu_packed(weight)
        if packed is not None:
            wl, layout = packed, LAYOUT_KN_SWIGLU
    elif weight.transpose(1, 2).is_contiguous():
        wl, layout = weight.transpose(1, 2), LAYOUT_NK
    else:
        wl, layout = weight.contiguous(), LAYOUT_KN
    ws = _f32(weight_scale)
    _check(ws.numel() == e * n, f"{name}: weight_scale must be [E, N]")
    m = a_rows.shape[0]
    xs = _f32(x_scale)
    _check(xs.numel() == m, f"{name}: x_scale must have M entries")
    gl = group_list.to(torch.int64).contiguous()
    _check(gl.numel() == e, f"{name}: group_list has {gl.numel()} entries, weight has {e} groups")
    y, ys = _gsq_gather_fake(x, a_rows, weight, weight_scale, x_scale, group_list)
    if m == 0:
        return y, ys
    xc, rc = x.contiguous(), a_rows.contiguous()
    nbytes = _lib.query("tai_grouped_matmul_swiglu_quant_workspace_size", m, n, e)
    wsp = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    _lib.call("tai_grouped_matmul_swiglu_quant_gather", _p(xc), xc.shape[0], _p(rc), _p(wl), m, k, n, e, layout,
              _p(gl), int(group_list_type), _p(ws), _p(xs), _p(y), _p(ys), _p(wsp), nbytes, _stream(xc))
    return y, ys


_define("grouped_matmul_swiglu_quant_gather(Tensor x, Tensor a_rows, Tensor weight, Tensor weight_scale, "
        "Tensor x_scale, Tensor group_list, *, int group_list_type=0) -> (Tensor, Tensor)",
        _gsq_gather_fake, _gsq_gather_cuda)
