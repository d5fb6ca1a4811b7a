"""torch.library ops of the fused MoE grouped GEMMs (libtai_kernels.so).

  npu_grouped_matmul_swiglu_quant_v2   .../ge_converter/custom/grouped_matmul_swiglu_quant_v2.py:86-166
  npu_grouped_matmul_finalize_routing  .../ge_converter/custom/grouped_matmul_finalize_routing.py:32-133

Both take the W8A8 weights of all experts stacked as [E, K, N] (or the transposed view of an
[E, N, K] tensor) and a device-resident group_list, like npu_grouped_matmul.
"""
from __future__ import annotations

import weakref

import torch

from . import _lib
from ._lib import DT_NONE, LAYOUT_KN, LAYOUT_KN_SWIGLU, LAYOUT_NK
from ._ops_impl import _DT, _check, _define, _f32, _on_gpu, _p, _stream


def _weight_layout(name, w3):
    _check(w3.dim() == 3 and w3.dtype == torch.int8, f"{name}: weight must be int8 [E, K, N]")
    if w3.is_contiguous():
        return w3, LAYOUT_KN
    if w3.transpose(1, 2).is_contiguous():
        return w3.transpose(1, 2), LAYOUT_NK
    return w3.contiguous(), LAYOUT_KN


# Gate / up interleaved copies of [E, K, N] SwiGLU weights (TAI_LAYOUT_KN_SWIGLU), made once per weight
# like the NPU's load-time format cast. Keyed by the weight's storage (address and shape), so aliases
# of one weight (a Parameter made from a tensor shares its storage and version counter) share one
# copy; an entry is dropped with the tensor that made it, and a weight written in place (its version
# moves) is packed anew.
_SWI_CACHE: dict = {}


def _swiglu_packed(w3: torch.Tensor):
    """The TAI_LAYOUT_KN_SWIGLU copy of the contiguous [E, K, N] weight w3, or None (N % 512 != 0,
    or under hipGraph capture before a warm-up made it: nothing is allocated during a capture)."""
    e, k, n = w3.shape
    if not w3.is_contiguous() or n % 512 != 0:
        return None
    key = (w3.data_ptr(), tuple(w3.shape), w3.device.index)
    ent = _SWI_CACHE.get(key)
    if ent is not None and ent[0]() is not None and ent[1] == w3._version:
        return ent[3]
    if torch.cuda.is_current_stream_capturing():
        return None
    packed = torch.empty_like(w3)
    _lib.call("tai_swiglu_pack_kn", _p(w3), e * k, n, _p(packed), _stream(w3))
    def drop(ref, key=key):
        if _SWI_CACHE.get(key, (None,))[0] is ref:  # not an entry made since by another tensor
            del _SWI_CACHE[key]

    _SWI_CACHE[key] = (weakref.ref(w3, drop), w3._version, None, packed)
    return packed


def _group_list(name, group_list, e, device):
    gl = group_list.to(torch.int64).contiguous() if isinstance(group_list, torch.Tensor) else \
        torch.tensor(list(group_list), dtype=torch.int64, device=device)
    _check(gl.numel() == e, f"{name}: group_list has {gl.numel()} entries, weight has {e} groups")
    return gl


# ============================================================================ swiglu_quant_v2
def _gsq_fake(x, weight, weight_scale, x_scale, group_list, *, smooth_scale=None, weight_assist_matrix=None,
              bias=None, dequant_mode=0, dequant_dtype=0, quant_mode=0, quant_dtype=1, group_list_type=0,
              tuning_config=None, x_dtype=None, weight_dtype=None, weight_scale_dtype=None, x_scale_dtype=None):
    n = weight[0].shape[-1]
    return (torch.empty([x.shape[0], n // 2], dtype=torch.int8, device=x.device),
            torch.empty([x.shape[0]], dtype=torch.float32, device=x.device))


def _gsq_cuda(x, weight, weight_scale, x_scale, group_list, *, smooth_scale=None, weight_assist_matrix=None,
              bias=None, dequant_mode=0, dequant_dtype=0, quant_mode=0, quant_dtype=1, group_list_type=0,
              tuning_config=None, x_dtype=None, weight_dtype=None, weight_scale_dtype=None, x_scale_dtype=None):
    """W8A8 grouped GEMM + dequant + silu(gate) * up + per-token int8 quantisation in one op."""
    name = "npu_grouped_matmul_swiglu_quant_v2"
    _on_gpu(x, x_scale, *weight, *weight_scale)
    _check(len(weight) == 1 and len(weight_scale) == 1, f"{name}: one stacked weight and weight_scale are supported")
    _check(not weight_assist_matrix, f"{name}: weight_assist_matrix is not supported")
    _check(dequant_mode in (None, 0) and quant_mode in (None, 0) and quant_dtype in (None, 1),
           f"{name}: only dequant_mode 0 with per-token int8 quantisation (quant_mode 0, quant_dtype 1) is supported")
    _check(x_dtype is None and weight_dtype is None and weight_scale_dtype is None and x_scale_dtype is None,
           f"{name}: only int8 x / weight with fp32 scales are supported")
    _check(group_list_type in (0, 1), f"{name}: group_list_type must be 0 (cumsum) or 1 (count)")
    _check(x.dtype == torch.int8 and x.dim() == 2, f"{name}: x must be int8 [M, K]")
    wl, layout = _weight_layout(name, weight[0])
    e, k, n = weight[0].shape
    _check(x.shape[1] == k and n % 2 == 0, f"{name}: x is [M, K] and the weight [E, K, N] with N even")
    if layout == LAYOUT_KN:
        packed = _swiglu_packed(wl)
        if packed is not None:
            wl, layout = packed, LAYOUT_KN_SWIGLU
    ws = _f32(weight_scale[0])
    _check(ws.numel() == e * n, f"{name}: weight_scale must be [E, N]")
    xs = _f32(x_scale)
    m = x.shape[0]
    _check(xs.numel() == m, f"{name}: x_scale must have M entries")
    gl = _group_list(name, group_list, e, x.device)
    if smooth_scale is not None or bias is not None:
        return _gsq_composed(name, x, weight[0], ws, xs, gl, group_list_type, smooth_scale, bias, e, n)
    y, ys = _gsq_fake(x, weight, weight_scale, x_scale, group_list)
    if m == 0:
        return y, ys
    xc = x.contiguous()
    nbytes = _lib.query("tai_grouped_matmul_swiglu_quant_workspace_size", m, n, e)
    wsp = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    _lib.call("tai_grouped_matmul_swiglu_quant", _p(xc), _p(wl), m, k, n, e, layout, _p(gl), int(group_list_type),
              _p(ws), _p(xs), _p(y), _p(ys), _p(wsp), nbytes, _stream(xc))
    return y, ys


def _gsq_composed(name, x, weight, ws, xs, gl, group_list_type, smooth_scale, bias, e, n):
    """smooth_scale and bias run the op as its two halves, both on the GPU kernels: the int32 grouped
    GEMM (npu_grouped_matmul) and npu_dequant_swiglu_quant with activate_left, dynamic quantisation,
    the bias (int32 added to the accumulators before the dequantisation, fp32 after it; [E, N]) and the
    smooth scale as its quant_scale (h * smooth_scale[group] before the per-row quantisation;
    [E, N/2] or [N/2] shared by the groups). The GE op takes both inputs
    (grouped_matmul_swiglu_quant_v2.py:146-161) without fixing their arithmetic; this is the fold's
    reading of them."""
    if smooth_scale is not None:
        sm = smooth_scale.to(torch.float32)
        _check(sm.numel() in (n // 2, e * n // 2), f"{name}: smooth_scale must be [E, N/2] or [N/2]")
        sm = sm.reshape(-1, n // 2).expand(e, n // 2).contiguous()
    else:
        sm = None
    if bias is not None:
        _check(bias.numel() == e * n and bias.dtype in (torch.int32, torch.float32, torch.float16, torch.bfloat16),
               f"{name}: bias must be [E, N] int32 or float")
        bias = bias.reshape(e, n)
    acc = torch.ops.npu.npu_grouped_matmul([x], [weight], group_list=gl, split_item=3, group_type=0,
                                           group_list_type=group_list_type, output_dtype=torch.int32)[0]
    counts = gl if group_list_type == 1 else torch.diff(gl, prepend=gl.new_zeros(1))
    return torch.ops.npu.npu_dequant_swiglu_quant(acc, weight_scale=ws.reshape(e, n), activation_scale=xs, bias=bias,
                                                  quant_scale=sm, group_index=counts, activate_left=True, quant_mode=1)


_define("npu", "npu_grouped_matmul_swiglu_quant_v2(Tensor x, Tensor[] weight, Tensor[] weight_scale, Tensor x_scale, "
               "Tensor group_list, *, Tensor? smooth_scale=None, Tensor[]? weight_assist_matrix=None, "
               "Tensor? bias=None, int? dequant_mode=0, int? dequant_dtype=0, int? quant_mode=0, "
               "int? quant_dtype=1, int? group_list_type=0, int[]? tuning_config=None, int? x_dtype=None, "
               "int? weight_dtype=None, int? weight_scale_dtype=None, int? x_scale_dtype=None) -> (Tensor, Tensor)",
        _gsq_fake, _gsq_cuda)


# ============================================================================ finalize_routing
def _gfr_fake(x, w, group_list, *, scale=None, bias=None, offset=None, pertoken_scale=None, shared_input=None,
              logit=None, row_index=None, dtype=None, shared_input_weight=1.0, shared_input_offset=0, output_bs=0,
              group_list_type=1, tuning_config=()):
    bs = output_bs if output_bs else x.shape[0]
    return torch.empty([bs, w.shape[-1]], dtype=torch.float32, device=x.device)


def _gfr_cuda(x, w, group_list, *, scale=None, bias=None, offset=None, pertoken_scale=None, shared_input=None,
              logit=None, row_index=None, dtype=None, shared_input_weight=1.0, shared_input_offset=0, output_bs=0,
              group_list_type=1, tuning_config=()):
    """W8A8 grouped GEMM + weighted combine of each token's rows into an fp32 output."""
    name = "npu_grouped_matmul_finalize_routing"
    _on_gpu(x, w, scale, bias, pertoken_scale, shared_input, logit, row_index)
    _check(dtype in (None, torch.float32), f"{name}: only fp32 output is supported (as the reference converter)")
    _check(offset is None, f"{name}: offset (int4 weights) is not supported")
    _check(x.dtype == torch.int8 and x.dim() == 2, f"{name}: x must be int8 [M, K]")
    _check(scale is not None, f"{name}: scale is required")
    _check(group_list_type in (None, 0, 1), f"{name}: group_list_type must be 0 (cumsum) or 1 (count)")
    wl, layout = _weight_layout(name, w)
    e, k, n = w.shape
    m = x.shape[0]
    _check(x.shape[1] == k and n % 8 == 0, f"{name}: x is [M, K], the weight [E, K, N] with N a multiple of 8")
    sc = _f32(scale)
    _check(sc.numel() == e * n, f"{name}: scale must be [E, N]")
    bi = _f32(bias)
    _check(bi is None or bi.numel() == e * n, f"{name}: bias must be [E, N]")
    pts, lg = _f32(pertoken_scale), _f32(logit)
    _check(pts is None or pts.numel() == m, f"{name}: pertoken_scale must have M entries")
    _check(lg is None or lg.numel() == m, f"{name}: logit must have M entries")
    ri = None
    if row_index is not None:
        _check(row_index.dtype in (torch.int32, torch.int64) and row_index.numel() == m,
               f"{name}: row_index must be int32/int64 with M entries")
        ri = row_index.contiguous()
    bs = int(output_bs) if output_bs else m
    sh = None
    rows_sh = 0
    if shared_input is not None:
        _check(shared_input.dtype == torch.bfloat16 and shared_input.dim() == 2 and shared_input.shape[1] == n,
               f"{name}: shared_input must be bf16 [S, N]")
        sh = shared_input.contiguous()
        rows_sh = sh.shape[0]
        _check(0 <= int(shared_input_offset or 0) and int(shared_input_offset or 0) + rows_sh <= bs,
               f"{name}: shared_input rows must lie inside the output")
    gl = _group_list(name, group_list, e, x.device)
    y = torch.empty([bs, n], dtype=torch.float32, device=x.device)
    if bs == 0:
        return y
    xc = x.contiguous()
    nbytes = _lib.query("tai_grouped_matmul_finalize_routing_workspace_size", m, n, e, bs)
    wsp = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    _lib.call("tai_grouped_matmul_finalize_routing", _p(xc), _p(wl), m, k, n, e, layout, _p(gl),
              1 if group_list_type is None else int(group_list_type), _p(sc), _p(pts), _p(bi), _p(lg), _p(ri),
              _DT[ri.dtype] if ri is not None else DT_NONE, _p(sh), rows_sh,
              1.0 if shared_input_weight is None else float(shared_input_weight), int(shared_input_offset or 0), bs,
              _p(y), _p(wsp), nbytes, _stream(xc))
    return y


_define("npu", "npu_grouped_matmul_finalize_routing(Tensor x, Tensor w, Tensor group_list, *, Tensor? scale=None, "
               "Tensor? bias=None, Tensor? offset=None, Tensor? pertoken_scale=None, Tensor? shared_input=None, "
               "Tensor? logit=None, Tensor? row_index=None, ScalarType? dtype=None, float? shared_input_weight=1.0, "
               "int? shared_input_offset=0, int? output_bs=0, int? group_list_type=1, int[] tuning_config=[]) "
               "-> Tensor",
        _gfr_fake, _gfr_cuda)
