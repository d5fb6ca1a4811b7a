"""torch.library registration of the torch_npu-style fused ops served by libtai_kernels.so.

Namespaces and schemas follow the ops TorchAir's converters accept:
  npu::          torch_npu fused ops (converters in
                 python/torchair/_ge_concrete_graph/ge_converter/custom/*.py)
  npu_inference:: gating / dequant_swiglu_quant twins
                 (python/torchair/_contrib/custom_torch_ops/auto_register_custom_torch_ops.py:42-191)
  air::          npu_fused_infer_attention_score with tensor sequence lengths
                 (python/torchair/ops/_npu_fused_infer_attention_score.py:14-34)
Each op has a fake (meta) implementation with the reference's output-shape rules and a
ROCm (``CUDA`` dispatch key) implementation that checks arguments, allocates outputs with
the caching allocator and calls the C ABI on the current stream. No CPU implementation is
registered here: calling these ops on CPU tensors raises.
"""
from __future__ import annotations

import math
import weakref
from typing import List, Optional, Sequence

import torch

from . import _lib
from ._lib import DT_BF16, DT_FP16, DT_FP32, DT_INT32, DT_INT64, DT_INT8, DT_NONE, LAYOUT_KN, LAYOUT_NK

_DT = {
    torch.uint8: 0, torch.int8: DT_INT8, torch.int16: 2, torch.int32: DT_INT32, torch.int64: DT_INT64,
    torch.float16: DT_FP16, torch.float32: DT_FP32, torch.bfloat16: DT_BF16,
}
_CODE_TO_DTYPE = {v: k for k, v in _DT.items()}


def scalar_type_code(v) -> Optional[int]:
    """ScalarType argument (torch.dtype or its integer code) -> integer code."""
    if v is None:
        return None
    if isinstance(v, torch.dtype):
        return _DT[v]
    return int(v)


def dtype_of_code(code: int) -> torch.dtype:
    if code not in _CODE_TO_DTYPE:
        raise ValueError(f"unsupported ScalarType code {code}")
    return _CODE_TO_DTYPE[code]


def _p(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _f32(t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    if t is None:
        return None
    return t.to(torch.float32).contiguous()


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _on_gpu(*ts):
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError("npu fused ops run on the ROCm device only; got a tensor on " + str(t.device))


LIBS = {
    "npu": torch.library.Library("npu", "FRAGMENT"),
    "npu_inference": torch.library.Library("npu_inference", "FRAGMENT"),
    "air": torch.library.Library("air", "FRAGMENT"),
}


def _define(ns: str, schema: str, fake, cuda, name: Optional[str] = None):
    lib = LIBS[ns]
    lib.define(schema)
    op_name = name or schema.split("(")[0]
    torch.library.register_fake(f"{ns}::{op_name}", fake, lib=lib)
    lib.impl(op_name, cuda, "CUDA")


# ============================================================================ npu_dynamic_quant
def _dq_scale_shape(input, quant_mode):
    return [1] if quant_mode == "pertensor" else list(input.shape[:-1])


def _dynamic_quant_fake(input, *, smooth_scales=None, group_index=None, dst_type=None, quant_mode="pertoken",
                        dst_type_max=0.0):
    return (torch.empty(input.shape, dtype=torch.int8, device=input.device),
            torch.empty(_dq_scale_shape(input, quant_mode), dtype=torch.float32, device=input.device))


def _dq_prepare(name, input, smooth_scales, group_index, dst_type, quant_mode):
    _on_gpu(input, smooth_scales, group_index)
    code = scalar_type_code(dst_type)
    _check(code in (None, DT_INT8), f"{name}: dst_type {dst_type} not supported (int8 only)")
    _check(quant_mode in (None, "pertoken", "pertensor"), f"{name}: quant_mode must be 'pertoken' or 'pertensor'")
    _check(input.dtype in (torch.bfloat16, torch.float16, torch.float32), f"{name}: input must be bf16, fp16 or fp32")
    _check(input.dim() >= 1, f"{name}: input must have at least one dim")
    x = input.contiguous()
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    sm = _f32(smooth_scales)
    ng = 0
    gi = None
    if sm is not None:
        if group_index is not None:
            _check(sm.dim() == 2 and sm.shape[1] == cols, f"{name}: smooth_scales must be [G, H] with group_index")
            gi = group_index.contiguous()
            _check(gi.dtype in (torch.int32, torch.int64) and gi.numel() == sm.shape[0],
                   f"{name}: group_index must be int32/int64 with G entries")
            ng = gi.numel()
        else:
            _check(sm.numel() == cols, f"{name}: smooth_scales must have H entries")
    return x, rows, cols, sm, gi, ng


def _dq_v2(name, x, rows, cols, sm, gi, ng, symmetric, quant_mode, dst_type_max):
    """ge.DynamicQuantV2 (npu_dynamic_quant.py:21-25 symmetric, :47-61 asymmetric)."""
    per_tensor = quant_mode == "pertensor"
    y = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    sshape = [1] if per_tensor else list(x.shape[:-1])
    scale = torch.empty(sshape, dtype=torch.float32, device=x.device)
    offset = None if symmetric else torch.empty(sshape, dtype=torch.float32, device=x.device)
    if rows == 0:
        if per_tensor:
            scale.zero_()
            if offset is not None:
                offset.zero_()
        return y, scale, offset
    ws_bytes = _lib.query("tai_dynamic_quant_v2_workspace_size", rows)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    _lib.call("tai_dynamic_quant_v2", _p(x), _DT[x.dtype], rows, cols, _p(sm), _p(gi),
              _DT[gi.dtype] if gi is not None else DT_NONE, ng, 1 if symmetric else 0, 1 if per_tensor else 0,
              float(dst_type_max or 0.0), _p(y), _p(scale), _p(offset), _p(ws), ws_bytes, _stream(x))
    return y, scale, offset


def _dynamic_quant_cuda(input, *, smooth_scales=None, group_index=None, dst_type=None, quant_mode="pertoken",
                        dst_type_max=0.0):
    """npu_dynamic_quant: symmetric int8 (npu_dynamic_quant.py:8-42). Per token with dst_type_max 0 is
    ge.DynamicQuant; per tensor, or a custom range, is ge.DynamicQuantV2 (is_symmetrical=True)."""
    x, rows, cols, sm, gi, ng = _dq_prepare("npu_dynamic_quant", input, smooth_scales, group_index, dst_type,
                                            quant_mode)
    if quant_mode == "pertensor" or not math.isclose(dst_type_max or 0.0, 0.0, abs_tol=1e-12):
        y, scale, _ = _dq_v2("npu_dynamic_quant", x, rows, cols, sm, gi, ng, True, quant_mode, dst_type_max)
        return y, scale
    y = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    scale = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
    if rows == 0:
        return y, scale
    _lib.call("tai_dynamic_quant", _p(x), _DT[x.dtype], rows, cols, _p(sm), _p(gi),
              _DT[gi.dtype] if gi is not None else DT_NONE, ng, _p(y), _p(scale), _stream(x))
    return y, scale


_define("npu", "npu_dynamic_quant(Tensor input, *, Tensor? smooth_scales=None, Tensor? group_index=None, "
               "ScalarType? dst_type=None, str? quant_mode=\"pertoken\", float dst_type_max=0.0) -> (Tensor, Tensor)",
        _dynamic_quant_fake, _dynamic_quant_cuda)


def _dynamic_quant_asym_fake(input, *, smooth_scales=None, group_index=None, dst_type=None, quant_mode="pertoken",
                             dst_type_max=0.0):
    sshape = _dq_scale_shape(input, quant_mode)
    return (torch.empty(input.shape, dtype=torch.int8, device=input.device),
            torch.empty(sshape, dtype=torch.float32, device=input.device),
            torch.empty(sshape, dtype=torch.float32, device=input.device))


def _dynamic_quant_asym_cuda(input, *, smooth_scales=None, group_index=None, dst_type=None, quant_mode="pertoken",
                             dst_type_max=0.0):
    """npu_dynamic_quant_asymmetric: ge.DynamicQuantV2 with is_symmetrical=False (npu_dynamic_quant.py:47-61)."""
    x, rows, cols, sm, gi, ng = _dq_prepare("npu_dynamic_quant_asymmetric", input, smooth_scales, group_index,
                                            dst_type, quant_mode)
    _check(math.isclose(dst_type_max or 0.0, 0.0, abs_tol=1e-12),
           "npu_dynamic_quant_asymmetric: dst_type_max is not supported (the range is the full int8 range)")
    return _dq_v2("npu_dynamic_quant_asymmetric", x, rows, cols, sm, gi, ng, False, quant_mode, 0.0)


_define("npu", "npu_dynamic_quant_asymmetric(Tensor input, *, Tensor? smooth_scales=None, Tensor? group_index=None, "
               "ScalarType? dst_type=None, str? quant_mode=\"pertoken\", float dst_type_max=0.0) "
               "-> (Tensor, Tensor, Tensor)",
        _dynamic_quant_asym_fake, _dynamic_quant_asym_cuda)


# ============================================================================ npu_dequant_swiglu_quant
_DSQ_SCHEMA = ("npu_dequant_swiglu_quant(Tensor x, *, Tensor? weight_scale=None, Tensor? activation_scale=None, "
               "Tensor? bias=None, Tensor? quant_scale=None, Tensor? quant_offset=None, Tensor? group_index=None, "
               "bool activate_left=False, int quant_mode=0, int? dst_type=None, int? round_mode=None, "
               "int? activate_dim=None, int swiglu_mode=0, float clamp_limit=7.0, float glu_alpha=1.702, "
               "float glu_bias=1.0) -> (Tensor, Tensor)")


def _dsq_fake(x, *, weight_scale=None, activation_scale=None, bias=None, quant_scale=None, quant_offset=None,
              group_index=None, activate_left=False, quant_mode=0, dst_type=None, round_mode=None, activate_dim=None,
              swiglu_mode=0, clamp_limit=7.0, glu_alpha=1.702, glu_bias=1.0):
    """Output shapes of auto_register_custom_torch_ops.py:155-191."""
    activate_dim = -1 if activate_dim is None else activate_dim
    sel = activate_dim if activate_dim >= 0 else activate_dim + x.dim()
    if x.dim() <= 1:
        raise RuntimeError("x dim should larger than 1")
    if sel < 0 or sel >= x.dim():
        raise RuntimeError("activate dim should less than x dim")
    if x.size(sel) % 2 != 0:
        raise RuntimeError("x last dim should be even")
    if quant_mode not in (0, 1):
        raise RuntimeError("quant_mode only support 0 or 1, but got " + str(quant_mode))
    y_size = [x.size(i) // 2 if i == sel else x.size(i) for i in range(x.dim())]
    return (torch.empty(y_size, dtype=torch.int8, device=x.device),
            torch.empty(y_size[:-1], dtype=torch.float32, device=x.device))


def _dsq_cuda(x, *, weight_scale=None, activation_scale=None, bias=None, quant_scale=None, quant_offset=None,
              group_index=None, activate_left=False, quant_mode=0, dst_type=None, round_mode=None, activate_dim=None,
              swiglu_mode=0, clamp_limit=7.0, glu_alpha=1.702, glu_bias=1.0):
    """npu_dequant_swiglu_quant (npu_dequant_swiglu_quant.py:5-47): quant_mode 1 (dynamic, per-row symmetric
    int8 of h * quant_scale) or 0 (static: clamp(rint(h * quant_scale + quant_offset)), scale output 0);
    swiglu_mode 0 (halves) or 1 (odd-even blocked columns, the clamped SwiGLU with clamp_limit, glu_alpha
    and glu_bias; experiment_ops.h:3786-3790)."""
    _on_gpu(x, weight_scale, activation_scale, bias, quant_scale, quant_offset, group_index)
    y, scale = _dsq_fake(x, activate_dim=activate_dim, quant_mode=quant_mode)
    _check(activate_dim in (None, -1, x.dim() - 1), "npu_dequant_swiglu_quant: only the last dim can be activated")
    _check(quant_mode in (0, 1), "npu_dequant_swiglu_quant: quant_mode must be 0 (static) or 1 (dynamic)")
    _check(quant_mode == 0 or quant_offset is None, "npu_dequant_swiglu_quant: quant_offset applies to the static mode")
    _check(quant_mode == 1 or quant_scale is not None, "npu_dequant_swiglu_quant: the static mode needs quant_scale")
    _check(dst_type in (None, 1), "npu_dequant_swiglu_quant: only int8 output (dst_type 1) is supported")
    _check(round_mode in (None, 0), "npu_dequant_swiglu_quant: only round_mode 0 (rint) is supported")
    _check(swiglu_mode in (0, 1), "npu_dequant_swiglu_quant: swiglu_mode must be 0 or 1")
    _check(x.dtype == torch.int32, "npu_dequant_swiglu_quant: x must be int32")
    xc = x.contiguous()
    n2 = xc.shape[-1]
    n = n2 // 2
    rows = xc.numel() // n2 if n2 else 0
    ng = group_index.numel() if group_index is not None else 1
    ws = _f32(weight_scale)
    if ws is not None:
        _check(ws.numel() == ng * n2, "npu_dequant_swiglu_quant: weight_scale must have G*2H entries")
    act = _f32(activation_scale)
    if act is not None:
        _check(act.numel() == rows, "npu_dequant_swiglu_quant: activation_scale must have one entry per row")
    bi = None
    bias_dt = DT_NONE
    if bias is not None:
        bi = bias.contiguous() if bias.dtype == torch.int32 else _f32(bias)
        bias_dt = _DT[bi.dtype]
        _check(bi.numel() == ng * n2, "npu_dequant_swiglu_quant: bias must have G*2H entries")
    qs = _f32(quant_scale)
    if qs is not None:
        if qs.numel() == n and ng > 1:  # one row of scales shared by every group
            qs = qs.reshape(1, n).expand(ng, n).contiguous()
        _check(qs.numel() == ng * n, "npu_dequant_swiglu_quant: quant_scale must have H or G*H entries")
    qo = _f32(quant_offset)
    if qo is not None:
        if qo.numel() == n and ng > 1:
            qo = qo.reshape(1, n).expand(ng, n).contiguous()
        _check(qo.numel() == ng * n, "npu_dequant_swiglu_quant: quant_offset must have H or G*H entries")
    gi = None
    if group_index is not None:
        gi = group_index.contiguous()
        _check(gi.dtype in (torch.int32, torch.int64), "npu_dequant_swiglu_quant: group_index must be int32/int64")
    if rows == 0:
        return y, scale
    if swiglu_mode == 1:
        _lib.call("tai_dequant_swiglu_quant_clamped", _p(xc), rows, n2, _p(ws), _p(act), _p(bi), bias_dt, _p(qs),
                  _p(qo), _p(gi), _DT[gi.dtype] if gi is not None else DT_NONE, ng, 1 if activate_left else 0,
                  int(quant_mode), float(clamp_limit), float(glu_alpha), float(glu_bias), _p(y), _p(scale), _stream(xc))
        return y, scale
    _lib.call("tai_dequant_swiglu_quant_static", _p(xc), rows, n2, _p(ws), _p(act), _p(bi), bias_dt, _p(qs),
              _p(qo), _p(gi), _DT[gi.dtype] if gi is not None else DT_NONE, ng, 1 if activate_left else 0,
              int(quant_mode), _p(y), _p(scale), _stream(xc))
    return y, scale


_define("npu", _DSQ_SCHEMA, _dsq_fake, _dsq_cuda)
_define("npu_inference", _DSQ_SCHEMA, _dsq_fake, _dsq_cuda)


# ============================================================================ npu_swiglu
def _swiglu_fake(x, dim=-1):
    d = dim % x.dim() if x.dim() else 0
    _check(x.dim() > 0 and x.shape[d] % 2 == 0, "npu_swiglu: the split dimension must have an even size")
    shape = list(x.shape)
    shape[d] //= 2
    return x.new_empty(shape)


def _swiglu_cuda(x, dim=-1):
    """npu_swiglu (.../custom/npu_swiglu.py:4-14): silu of the first half of `dim` times the second half."""
    _on_gpu(x)
    _check(x.dtype in (torch.bfloat16, torch.float16, torch.float32), "npu_swiglu: x must be bf16, fp16 or fp32")
    y = _swiglu_fake(x, dim)
    d = dim % x.dim()
    xc = x.contiguous()
    outer = math.prod(xc.shape[:d])
    inner = math.prod(xc.shape[d + 1:])
    n = xc.shape[d] // 2
    if y.numel():
        _lib.call("tai_swiglu", _p(xc), _DT[xc.dtype], outer, n, inner, _p(y), _stream(xc))
    return y


_define("npu", "npu_swiglu(Tensor self, int dim=-1) -> Tensor", _swiglu_fake, _swiglu_cuda)


# ============================================================================ npu_moe_compute_expert_tokens
def _cet_fake(sorted_experts, num_experts):
    return sorted_experts.new_empty((num_experts,), dtype=torch.int32)


def _cet_cuda(sorted_experts, num_experts):
    """npu_moe_compute_expert_tokens (.../custom/npu_moe_compute_expert_tokens.py:4-11): the end row of each
    expert in the ascending expert ids of the legacy routing."""
    _on_gpu(sorted_experts)
    _check(sorted_experts.dtype == torch.int32, "npu_moe_compute_expert_tokens: sorted_experts must be int32")
    _check(0 < num_experts < 2147483647, "npu_moe_compute_expert_tokens: num_experts must be positive")
    se = sorted_experts.contiguous()
    out = _cet_fake(se, num_experts)
    _lib.call("tai_moe_compute_expert_tokens", _p(se), se.numel(), num_experts, _p(out), _stream(se))
    return out


_define("npu", "npu_moe_compute_expert_tokens(Tensor sorted_experts, int num_experts) -> Tensor", _cet_fake, _cet_cuda)


# ============================================================================ npu_quant_matmul
def _qmm_out_dtype(output_dtype) -> torch.dtype:
    code = scalar_type_code(output_dtype)
    if code is None or code == DT_INT8:
        return torch.int8
    return dtype_of_code(code)


def _qmm_fake(x1, x2, scale, *, offset=None, pertoken_scale=None, bias=None, output_dtype=None, x1_dtype=None,
              x2_dtype=None, pertoken_scale_dtype=None, scale_dtype=None, group_sizes=None):
    shape = list(x1.shape[:-1]) + [x2.shape[-1]]
    return torch.empty(shape, dtype=_qmm_out_dtype(output_dtype), device=x1.device)


# [N, K] copies of [K, N] int8 weights, made once per weight (the NPU's counterpart is the format cast
# of weights at load time). Keyed by the tensor object; an entry is dropped with its weight, and a
# weight written in place (its version moves) or moved to another address is transposed anew.
_NK_CACHE: dict = {}


def _prepacked_nk(w: torch.Tensor, m: int):
    """[N, K] storage of the contiguous [K, N] int8 weight w when a product of m rows takes the [N, K]
    kernel (tall products), else None."""
    k, n = w.shape
    if not w.is_contiguous() or not _lib.query("tai_quant_matmul_prepack_wanted", m, k, n):
        return None
    key = id(w)
    ent = _NK_CACHE.get(key)
    if ent is not None and ent[0]() is w and ent[1] == w._version and ent[2] == w.data_ptr():
        return ent[3]
    if torch.cuda.is_current_stream_capturing():
        return None  # no allocation inside a capture: the kernel transposes into its workspace
    nk = torch.empty((n, k), dtype=torch.int8, device=w.device)
    _lib.call("tai_transpose_kn_to_nk", _p(w), k, n, _p(nk), _stream(w))
    _NK_CACHE[key] = (weakref.ref(w, lambda _r, key=key: _NK_CACHE.pop(key, None)), w._version, w.data_ptr(), nk)
    return nk


def _weight_layout(w: torch.Tensor):
    """Returns (tensor, layout) with the last two dims either [K,N] row-major or a [N,K] row-major storage."""
    if w.is_contiguous():
        return w, LAYOUT_KN
    wt = w.transpose(-1, -2)
    if wt.is_contiguous():
        return wt, LAYOUT_NK
    return w.contiguous(), LAYOUT_KN


def _qmm_cuda(x1, x2, scale, *, offset=None, pertoken_scale=None, bias=None, output_dtype=None, x1_dtype=None,
              x2_dtype=None, pertoken_scale_dtype=None, scale_dtype=None, group_sizes=None):
    """npu_quant_matmul W8A8 (quantmatmul.py:63-255)."""
    _on_gpu(x1, x2, scale, pertoken_scale, bias)
    _check(x1.dtype == torch.int8 and x2.dtype == torch.int8, "npu_quant_matmul: x1 and x2 must be int8")
    _check(x2.dim() == 2, "npu_quant_matmul: x2 must be 2-D [K, N]")
    _check(group_sizes is None, "npu_quant_matmul: group_sizes is not supported")
    out_dtype = _qmm_out_dtype(output_dtype)
    _check(out_dtype in (torch.int8, torch.int32, torch.bfloat16, torch.float16, torch.float32),
           "npu_quant_matmul: output_dtype must be int8, int32, bf16, fp16 or fp32")
    _check(offset is None or out_dtype == torch.int8, "npu_quant_matmul: offset applies to int8 output only")
    k = x1.shape[-1]
    _check(x2.shape[0] == k, f"npu_quant_matmul: K mismatch {k} vs {x2.shape[0]}")
    n = x2.shape[1]
    a = x1.contiguous()
    m = a.numel() // k if k else 0
    w, layout = _weight_layout(x2)
    if layout == LAYOUT_KN:
        nk = _prepacked_nk(w, m)
        if nk is not None:
            w, layout = nk, LAYOUT_NK
    # npu_trans_quant_param packs an fp32 scale (and offset) into int64 words; converting those words
    # numerically would give meaningless scales, so they are refused
    _check(scale is None or scale.dtype not in (torch.int64, torch.uint64),
           "npu_quant_matmul: packed int64 scales are not supported; pass fp32")
    sc = _f32(scale) if scale is not None else None
    if sc is not None:
        _check(sc.numel() in (1, n), "npu_quant_matmul: scale must have 1 or N entries")
    pts = _f32(pertoken_scale)
    if pts is not None:
        _check(pts.numel() == m, "npu_quant_matmul: pertoken_scale must have M entries")
    bi = None
    bias_dt = DT_NONE
    if bias is not None:
        bi = bias.contiguous() if bias.dtype == torch.int32 else _f32(bias)
        bias_dt = _DT[bi.dtype]
        _check(bi.numel() == n, "npu_quant_matmul: bias must have N entries")
    out = torch.empty(list(x1.shape[:-1]) + [n], dtype=out_dtype, device=x1.device)
    if m == 0 or n == 0:
        return out
    if k == 0:
        return out.zero_()
    off = _f32(offset)
    if off is not None:
        _check(off.numel() in (1, n), "npu_quant_matmul: offset must have 1 or N entries")
    ws_bytes = _lib.query("tai_quant_matmul_workspace_size", m, k, n, _DT[out_dtype])
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x1.device) if ws_bytes else None
    _lib.call("tai_quant_matmul", _p(a), _p(w), m, k, n, layout, _p(sc), sc.numel() if sc is not None else 0,
              _p(off), off.numel() if off is not None else 0, _p(pts), _p(bi), bias_dt, _DT[out_dtype], _p(out),
              _p(ws), ws_bytes, _stream(a))
    return out


_define("npu", "npu_quant_matmul(Tensor x1, Tensor x2, Tensor scale, *, Tensor? offset=None, "
               "Tensor? pertoken_scale=None, Tensor? bias=None, ScalarType? output_dtype=None, "
               "ScalarType? x1_dtype=None, ScalarType? x2_dtype=None, ScalarType? pertoken_scale_dtype=None, "
               "ScalarType? scale_dtype=None, int[]? group_sizes=None) -> Tensor",
        _qmm_fake, _qmm_cuda)


# ============================================================================ npu_grouped_matmul
_GMM_TAIL = ("*, Tensor[]? bias=None, Tensor[]? scale=None, Tensor[]? offset=None, Tensor[]? antiquant_scale=None, "
             "Tensor[]? antiquant_offset=None, Tensor[]? per_token_scale=None, {gl}, "
             "Tensor[]? activation_input=None, Tensor[]? activation_quant_scale=None, "
             "Tensor[]? activation_quant_offset=None, int? split_item=0, int? group_type=None, "
             "int? group_list_type=0, int? act_type=0, int[]? tuning_config=None, ScalarType? output_dtype=None"
             ") -> Tensor[]")


def _gmm_out_dtype(x, output_dtype):
    code = scalar_type_code(output_dtype)
    if code is None:
        return torch.int8 if x[0].dtype == torch.int8 else x[0].dtype
    return dtype_of_code(code)


def _gmm_group_rows(group_list, group_list_type, e):
    """Host list of the rows of each group (cumulative ends or counts)."""
    vals = [int(v) for v in (group_list.tolist() if isinstance(group_list, torch.Tensor) else group_list)]
    _check(len(vals) == e, f"npu_grouped_matmul: group_list has {len(vals)} entries for {e} groups")
    if group_list_type == 1:
        return vals
    out, prev = [], 0
    for v in vals:
        out.append(max(v - prev, 0))
        prev = max(prev, v)
    return out


def _gmm_pairs(x, weight):
    """Multi-tensor form: one x per group (group_list absent); weights as a list or one stacked tensor."""
    ws = list(weight) if len(weight) > 1 else ([weight[0]] if weight[0].dim() == 2 else list(weight[0].unbind(0)))
    _check(len(ws) == len(x), f"npu_grouped_matmul: {len(x)} x tensors need {len(x)} weights, got {len(ws)}")
    return ws


def _gmm_fake(x, weight, *, bias=None, scale=None, offset=None, antiquant_scale=None, antiquant_offset=None,
              per_token_scale=None, group_list=None, activation_input=None, activation_quant_scale=None,
              activation_quant_offset=None, split_item=0, group_type=None, group_list_type=0, act_type=0,
              tuning_config=None, output_dtype=None):
    od = _gmm_out_dtype(x, output_dtype)
    dev = x[0].device
    if group_list is None:  # per-group pairs
        ws = _gmm_pairs(x, weight)
        outs = [torch.empty([xi.shape[0], wi.shape[-1]], dtype=od, device=dev) for xi, wi in zip(x, ws)]
        if split_item in (2, 3):
            return [torch.empty([sum(o.shape[0] for o in outs), outs[0].shape[1]], dtype=od, device=dev)]
        return outs
    n = weight[0].shape[-1]
    m = x[0].shape[0]
    if split_item in (0, 1):
        _check(not isinstance(group_list, torch.Tensor),
               "npu_grouped_matmul: split_item 0/1 with groups along M need a list-valued group_list to trace "
               "(the output shapes depend on it)")
        rows = _gmm_group_rows(group_list, group_list_type, len(group_list))
        return [torch.empty([r, n], dtype=od, device=dev) for r in rows]
    return [torch.empty([m, n], dtype=od, device=dev)]


def _gmm_cuda(x, weight, *, bias=None, scale=None, offset=None, antiquant_scale=None, antiquant_offset=None,
              per_token_scale=None, group_list=None, activation_input=None, activation_quant_scale=None,
              activation_quant_offset=None, split_item=0, group_type=None, group_list_type=0, act_type=0,
              tuning_config=None, output_dtype=None):
    """npu_grouped_matmul int8 path (grouped_matmul.py:210-365): one x with groups along M (group_type 0,
    group_list given), or one x per group (group_list absent); split_item 0/1 return one output per group,
    2/3 one output over all rows."""
    _check(split_item in (0, 1, 2, 3), "npu_grouped_matmul: split_item must be 0, 1, 2 or 3")
    _check(not (offset or antiquant_scale or antiquant_offset or activation_input or activation_quant_scale
                or activation_quant_offset), "npu_grouped_matmul: offset/antiquant/activation inputs are not supported")
    _check(act_type in (None, 0), "npu_grouped_matmul: act_type must be 0")
    _check(group_list_type in (0, 1), "npu_grouped_matmul: group_list_type must be 0 (cumsum) or 1 (count)")
    if group_list is None:
        return _gmm_pairs_cuda(x, weight, bias, scale, per_token_scale, split_item, output_dtype)
    _check(len(x) == 1, "npu_grouped_matmul: with a group_list, x is a single [M, K] tensor")
    _check(group_type in (None, 0), "npu_grouped_matmul: only group_type 0 (groups along M) is supported")
    xt = x[0]
    _on_gpu(xt, *weight)
    _check(xt.dtype == torch.int8, "npu_grouped_matmul: only the int8 (W8A8) path is supported")
    if len(weight) == 1:
        w3 = weight[0]
        _check(w3.dim() == 3, "npu_grouped_matmul: stacked weight must be [E, K, N]")
    else:
        w3 = torch.stack(list(weight))
    _check(w3.dtype == torch.int8, "npu_grouped_matmul: weight must be int8")
    e, k, n = w3.shape
    _check(xt.dim() == 2 and xt.shape[1] == k, "npu_grouped_matmul: x must be [M, K] with K matching the weight")
    out_dtype = _gmm_out_dtype(x, output_dtype)
    _check(out_dtype in (torch.int32, torch.bfloat16, torch.float16, torch.float32),
           "npu_grouped_matmul: output_dtype must be int32, bf16, fp16 or fp32 for int8 inputs")
    if isinstance(group_list, torch.Tensor):
        gl = group_list.to(torch.int64).contiguous()
    else:
        gl = torch.tensor(list(group_list), dtype=torch.int64, device=xt.device)
    _check(gl.numel() == e, f"npu_grouped_matmul: group_list has {gl.numel()} entries, weight has {e} groups")
    if w3.is_contiguous():
        wl, layout = w3, LAYOUT_KN
    elif w3.transpose(1, 2).is_contiguous():
        wl, layout = w3.transpose(1, 2), LAYOUT_NK
    else:
        wl, layout = w3.contiguous(), LAYOUT_KN
    sc = None
    if scale:
        _check(all(t.dtype not in (torch.int64, torch.uint64) for t in scale),
               "npu_grouped_matmul: packed int64 scales are not supported; pass fp32")
        sc = _f32(scale[0] if len(scale) == 1 else torch.stack(list(scale)))
        _check(sc.numel() == e * n, "npu_grouped_matmul: scale must be [E, N]")
    pts = _f32(per_token_scale[0]) if per_token_scale else None
    m = xt.shape[0]
    if pts is not None:
        _check(pts.numel() == m, "npu_grouped_matmul: per_token_scale must have M entries")
    bi = None
    bias_dt = DT_NONE
    if bias:
        b = bias[0] if len(bias) == 1 else torch.stack(list(bias))
        bi = b.contiguous() if b.dtype == torch.int32 else _f32(b)
        bias_dt = _DT[bi.dtype]
        _check(bi.numel() == e * n, "npu_grouped_matmul: bias must be [E, N]")
    _check(out_dtype == torch.int32 or sc is not None, "npu_grouped_matmul: floating output needs scale")
    xc = xt.contiguous()
    out = torch.empty([m, n], dtype=out_dtype, device=xt.device)
    if m > 0 and n > 0:
        ws_bytes = _lib.query("tai_grouped_matmul_workspace_size", m, n, e)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=xt.device)
        _lib.call("tai_grouped_matmul", _p(xc), _p(wl), m, k, n, e, layout, _p(gl), int(group_list_type), _p(sc),
                  _p(pts), _p(bi), bias_dt, _DT[out_dtype], _p(out), _p(ws), ws_bytes, _stream(xc))
    if split_item in (2, 3):
        return [out]
    # one output per group: the rows of each group (the split needs the group sizes on the host)
    rows = _gmm_group_rows(group_list, group_list_type, e)
    outs, r0 = [], 0
    for r in rows:
        r = min(r, m - r0)
        outs.append(out[r0:r0 + r].clone())
        r0 += r
    return outs


def _gmm_pairs_cuda(x, weight, bias, scale, per_token_scale, split_item, output_dtype):
    """One x per group: y_i = x_i @ w_i with group i's scale and bias; per_token_scale holds the rows of
    all groups in order. Each pair runs the dense W8A8 GEMM."""
    ws = _gmm_pairs(x, weight)
    g = len(x)
    out_dtype = _gmm_out_dtype(x, output_dtype)
    _check(out_dtype in (torch.int32, torch.bfloat16, torch.float16, torch.float32),
           "npu_grouped_matmul: output_dtype must be int32, bf16, fp16 or fp32 for int8 inputs")

    def per_group(lst, name):
        if not lst:
            return [None] * g
        if len(lst) == g:
            return list(lst)
        _check(len(lst) == 1 and lst[0].dim() == 2 and lst[0].shape[0] == g,
               f"npu_grouped_matmul: {name} must hold one tensor per group or one stacked [G, N] tensor")
        return list(lst[0].unbind(0))

    scs, bis = per_group(scale, "scale"), per_group(bias, "bias")
    pts_all = _f32(per_token_scale[0]) if per_token_scale else None
    _check(out_dtype == torch.int32 or all(s is not None for s in scs), "npu_grouped_matmul: floating output needs scale")
    outs, r0 = [], 0
    for xi, wi, si, bi in zip(x, ws, scs, bis):
        _check(xi.dtype == torch.int8 and wi.dtype == torch.int8, "npu_grouped_matmul: only the int8 (W8A8) path is "
                                                                  "supported")
        _check(wi.dim() == 2 and xi.shape[-1] == wi.shape[0], "npu_grouped_matmul: x_i [M_i, K] needs w_i [K, N_i]")
        rows = xi.numel() // xi.shape[-1] if xi.shape[-1] else 0
        pts = pts_all[r0:r0 + rows] if pts_all is not None else None
        r0 += rows
        one = torch.ones(1, device=xi.device)
        outs.append(_qmm_cuda(xi, wi, si if si is not None else one, pertoken_scale=pts, bias=bi,
                              output_dtype=out_dtype))
    if split_item in (2, 3):
        return [torch.cat([o.reshape(-1, o.shape[-1]) for o in outs], 0)]
    return outs


_define("npu", "npu_grouped_matmul(Tensor[] x, Tensor[] weight, " + _GMM_TAIL.format(gl="Tensor? group_list=None"),
        _gmm_fake, _gmm_cuda)
LIBS["npu"].define("npu_grouped_matmul.List(Tensor[] x, Tensor[] weight, " +
                   _GMM_TAIL.format(gl="int[]? group_list=None"))
torch.library.register_fake("npu::npu_grouped_matmul.List", _gmm_fake, lib=LIBS["npu"])
LIBS["npu"].impl("npu_grouped_matmul.List", _gmm_cuda, "CUDA")


# ============================================================================ npu_moe_gating_top_k
_GATE_SCHEMA = ("npu_moe_gating_top_k(Tensor x, int k, *, Tensor? bias=None, int k_group=1, int group_count=1, "
                "int group_select_mode=0, int renorm=0, int norm_type=0, bool out_flag=False, "
                "float routed_scaling_factor=1.0, float eps=1e-20) -> (Tensor, Tensor, Tensor)")


def _gate_fake(x, k, *, bias=None, k_group=1, group_count=1, group_select_mode=0, renorm=0, norm_type=0,
               out_flag=False, routed_scaling_factor=1.0, eps=1e-20):
    """Output shapes of auto_register_custom_torch_ops.py:103-114."""
    return (x.new_empty((x.size(0), k), dtype=x.dtype), x.new_empty((x.size(0), k), dtype=torch.int32),
            x.new_empty((x.size(0), x.size(1)), dtype=torch.float32))


def _gate_cuda(x, k, *, bias=None, k_group=1, group_count=1, group_select_mode=0, renorm=0, norm_type=0,
               out_flag=False, routed_scaling_factor=1.0, eps=1e-20):
    """npu_moe_gating_top_k (npu_moe_gating_top_k.py:4-22)."""
    _on_gpu(x, bias)
    _check(x.dim() == 2, "npu_moe_gating_top_k: x must be [T, E]")
    y, idx, out = _gate_fake(x, k)
    xc = x.contiguous()
    bc = bias.contiguous() if bias is not None else None
    if bc is not None:
        _check(bc.numel() == x.shape[1], "npu_moe_gating_top_k: bias must have E entries")
    if x.shape[0] == 0:
        return y, idx, out
    _lib.call("tai_moe_gating_top_k", _p(xc), _DT[xc.dtype], xc.shape[0], xc.shape[1], int(k), _p(bc),
              _DT[bc.dtype] if bc is not None else DT_NONE, int(k_group), int(group_count), int(group_select_mode),
              int(renorm), int(norm_type), 1 if out_flag else 0, float(routed_scaling_factor), float(eps), _p(y),
              _p(idx), _p(out), _stream(xc))
    return y, idx, out


_define("npu", _GATE_SCHEMA, _gate_fake, _gate_cuda)
_define("npu_inference", _GATE_SCHEMA, _gate_fake, _gate_cuda)


# ============================================================================ npu_moe_init_routing(_v2)
LEGACY_ROUTING_EXPERT_BINS = 1024  # legacy init_routing carries no expert count: ids must be < 1024


def _init_routing_fake(x, row_idx, expert_idx, active_num):
    t, k = expert_idx.shape
    rows = min(t, active_num) * k if active_num >= 0 else t * k
    return (x.new_empty((rows, x.shape[1])), x.new_empty((t * k,), dtype=torch.int32),
            x.new_empty((t * k,), dtype=torch.int32))


def _init_routing_cuda(x, row_idx, expert_idx, active_num):
    """npu_moe_init_routing (moe_init_routing.py:10-21)."""
    _on_gpu(x, row_idx, expert_idx)
    _check(x.dim() == 2 and expert_idx.dim() == 2 and row_idx.shape == expert_idx.shape,
           "npu_moe_init_routing: x [T,H], row_idx and expert_idx [T,k]")
    _check(row_idx.dtype == torch.int32 and expert_idx.dtype == torch.int32,
           "npu_moe_init_routing: row_idx and expert_idx must be int32")
    ex, ri, ei = _init_routing_fake(x, row_idx, expert_idx, active_num)
    t, k = expert_idx.shape
    if t == 0:
        return ex, ri, ei
    xc, rc, ec = x.contiguous(), row_idx.contiguous(), expert_idx.contiguous()
    bins = LEGACY_ROUTING_EXPERT_BINS
    ws_bytes = _lib.query("tai_moe_init_routing_workspace_size", t, k, bins)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    _lib.call("tai_moe_init_routing", _p(xc), xc.element_size(), t, xc.shape[1], _p(rc), _p(ec), k, bins,
              ex.shape[0], _p(ex), _p(ri), _p(ei), _p(ws), ws_bytes, _stream(xc))
    return ex, ri, ei


_define("npu", "npu_moe_init_routing(Tensor x, Tensor row_idx, Tensor expert_idx, int active_num) "
               "-> (Tensor, Tensor, Tensor)", _init_routing_fake, _init_routing_cuda)


def _v2_expert_range(expert_num, active_expert_range):
    if active_expert_range:
        lo, hi = int(active_expert_range[0]), int(active_expert_range[1])
    else:
        lo, hi = 0, int(expert_num)
    return lo, hi


def _init_routing_v2_fake(x, expert_idx, *, scale=None, offset=None, active_num=-1, expert_capacity=-1,
                          expert_num=-1, drop_pad_mode=0, expert_tokens_num_type=0, expert_tokens_num_flag=False,
                          quant_mode=-1, active_expert_range=(), row_idx_type=0):
    t, k = expert_idx.shape
    n = t * k
    lo, hi = _v2_expert_range(expert_num, active_expert_range)
    if drop_pad_mode == 1:  # expert e owns rows [e * capacity, (e + 1) * capacity)
        rows = max(hi - lo, 0) * max(expert_capacity, 0)
    else:
        rows = n if (active_num is None or active_num <= 0 or active_num >= n) else active_num
    quant = quant_mode in (0, 1)
    # expanded_scale: the gathered scale (unquantised), the per-row scale (dynamic); none for static
    n_scale = rows if ((scale is not None and quant_mode == -1) or quant_mode == 1) else 0
    return (x.new_empty((rows, x.shape[1]), dtype=torch.int8 if quant else x.dtype),
            x.new_empty((n,), dtype=torch.int32),
            x.new_empty((max(hi - lo, 0),), dtype=torch.int64),
            x.new_empty((n_scale,), dtype=torch.float32))


def _route_v2(x, expert_idx, scale, active_num, expert_capacity, expert_num, drop_pad_mode, expert_tokens_num_type,
              active_expert_range, row_idx_type):
    """Routing without quantisation: (expanded_x, expanded_row_idx, expert_tokens, expanded_scale)."""
    _check(expert_tokens_num_type in (0, 1), "npu_moe_init_routing_v2: expert_tokens_num_type must be 0 or 1")
    _check(x.dim() == 2 and expert_idx.dim() == 2 and expert_idx.shape[0] == x.shape[0],
           "npu_moe_init_routing_v2: x [T,H] and expert_idx [T,k]")
    _check(expert_idx.dtype == torch.int32, "npu_moe_init_routing_v2: expert_idx must be int32")
    lo, hi = _v2_expert_range(expert_num, active_expert_range)
    _check(hi > lo >= 0, "npu_moe_init_routing_v2: expert_num or active_expert_range is required")
    if drop_pad_mode == 1:
        _check(expert_capacity is not None and expert_capacity > 0,
               "npu_moe_init_routing_v2: drop_pad_mode 1 needs expert_capacity > 0")
    ex, ri, tok, es = _init_routing_v2_fake(x, expert_idx, scale=scale, active_num=active_num,
                                            expert_capacity=expert_capacity, expert_num=expert_num,
                                            drop_pad_mode=drop_pad_mode, active_expert_range=active_expert_range)
    t, k = expert_idx.shape
    xc, ec = x.contiguous(), expert_idx.contiguous()
    sc = _f32(scale)
    if sc is not None:
        _check(sc.numel() == t, "npu_moe_init_routing_v2: scale must have T entries")
    if drop_pad_mode == 1:
        ws_bytes = _lib.query("tai_moe_init_routing_v2_droppad_workspace_size", t, k, hi - lo, expert_capacity)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
        _lib.call("tai_moe_init_routing_v2_droppad", _p(xc), xc.element_size(), t, xc.shape[1], _p(ec), k, _p(sc),
                  expert_capacity, lo, hi, int(expert_tokens_num_type), _p(ex), _p(ri), _p(tok),
                  _p(es) if sc is not None else None, _p(ws), ws_bytes, _stream(xc))
        return ex, ri, tok, es
    if t == 0:
        return ex, ri, tok.zero_(), es
    ws_bytes = _lib.query("tai_moe_init_routing_workspace_size", t, k, hi - lo)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    _lib.call("tai_moe_init_routing_v2", _p(xc), xc.element_size(), t, xc.shape[1], _p(ec), k, _p(sc), ex.shape[0],
              lo, hi, int(expert_tokens_num_type), int(row_idx_type), _p(ex), _p(ri), _p(tok),
              _p(es) if sc is not None else None, _p(ws), ws_bytes, _stream(xc))
    return ex, ri, tok, es


def _group_ends(tok, expert_tokens_num_type, drop_pad_mode, capacity, n_groups, device):
    """Cumulative row ends of the experts' row blocks of expanded_x (int64, on the device)."""
    if drop_pad_mode == 1:
        return torch.arange(1, n_groups + 1, dtype=torch.int64, device=device) * capacity
    return tok if expert_tokens_num_type == 0 else torch.cumsum(tok, 0)


def _init_routing_v2_cuda(x, expert_idx, *, scale=None, offset=None, active_num=-1, expert_capacity=-1,
                          expert_num=-1, drop_pad_mode=0, expert_tokens_num_type=0, expert_tokens_num_flag=False,
                          quant_mode=-1, active_expert_range=(), row_idx_type=0):
    """npu_moe_init_routing_v2 (npu_moe_init_routing_v2.py:41-91; prototype experiment_ops.h:2138-2190).

    drop_pad_mode 0 (dropless) or 1 (dropPad with expert_capacity: expert e owns rows
    [e * capacity, (e + 1) * capacity), slots past the capacity are dropped, unfilled rows are zero).
    quant_mode -1: no quantisation (scale [T], if given, is gathered into expanded_scale).
    quant_mode 1 (dynamic) without scale: every expanded row is the symmetric per-row int8 quantisation
    of its token row and expanded_scale holds that row's scale; a token row and its copies quantise
    identically, so the T token rows are quantised once (the npu_dynamic_quant kernel) and the int8
    rows and scales are gathered. With a smooth scale ([1, H] or [E, H]) each expanded row is x * smooth
    of its expert, then quantised per row (npu_dynamic_quant with the experts' row blocks as groups).
    quant_mode 0 (static): y = clamp(rint(x * scale + offset)) with scale / offset of [1], [E, 1],
    [1, H] or [E, H] (per expert, per channel); no expanded_scale."""
    _on_gpu(x, expert_idx, scale, offset)
    _check(drop_pad_mode in (0, 1), "npu_moe_init_routing_v2: drop_pad_mode must be 0 (dropless) or 1 (dropPad)")
    _check(quant_mode in (-1, 0, 1), "npu_moe_init_routing_v2: quant_mode -1 (none), 0 (static) or 1 (dynamic) is "
           "supported")
    lo, hi = _v2_expert_range(expert_num, active_expert_range)
    n_e = hi - lo
    h = x.shape[-1]
    route = dict(active_num=active_num, expert_capacity=expert_capacity, expert_num=expert_num,
                 drop_pad_mode=drop_pad_mode, expert_tokens_num_type=expert_tokens_num_type,
                 active_expert_range=active_expert_range, row_idx_type=row_idx_type)
    if quant_mode == 1 and scale is None:
        _check(offset is None, "npu_moe_init_routing_v2: quant_mode 1 takes no offset")
        _check(x.dim() == 2, "npu_moe_init_routing_v2: x [T,H] and expert_idx [T,k]")
        q, s = torch.ops.npu.npu_dynamic_quant(x)
        return _route_v2(q, expert_idx, s, **route)
    if quant_mode == 1:  # smooth scales per expert (or shared), then per-row dynamic quantisation
        _check(offset is None, "npu_moe_init_routing_v2: quant_mode 1 takes no offset")
        sm = _f32(scale)
        _check(sm.numel() in (h, n_e * h), "npu_moe_init_routing_v2: the smooth scale must be [1, H] or [E, H]")
        ex, ri, tok, _ = _route_v2(x, expert_idx, None, **route)
        if sm.numel() == h:
            q, s = torch.ops.npu.npu_dynamic_quant(ex, smooth_scales=sm.reshape(h))
        else:
            ends = _group_ends(tok, expert_tokens_num_type, drop_pad_mode, expert_capacity, n_e, x.device)
            q, s = torch.ops.npu.npu_dynamic_quant(ex, smooth_scales=sm.reshape(n_e, h), group_index=ends)
        return q, ri, tok, s
    if quant_mode == 0:
        _check(scale is not None, "npu_moe_init_routing_v2: quant_mode 0 (static) needs scale")
        sc = _f32(scale)
        ofs = _f32(offset)
        # [1] per tensor, [H] / [1, H] per channel, [E, 1] per expert, [E, H] per expert and channel
        if scale.dim() >= 2:
            groups, cols = scale.numel() // scale.shape[-1], scale.shape[-1]
        else:
            groups, cols = 1, scale.numel()
        _check(groups in (1, n_e) and cols in (1, h), "npu_moe_init_routing_v2: static scale must be [1], [H], [1, H], "
               "[E, 1] or [E, H]")
        _check(ofs is None or ofs.numel() == sc.numel(), "npu_moe_init_routing_v2: offset must match scale")
        per_col = 1 if (cols == h and h != 1) else 0
        ex, ri, tok, _ = _route_v2(x, expert_idx, None, **route)
        y = torch.empty(ex.shape, dtype=torch.int8, device=x.device)
        ends = None
        if groups > 1 and drop_pad_mode == 0:
            ends = _group_ends(tok, expert_tokens_num_type, 0, 0, n_e, x.device)
        _lib.call("tai_static_quant_rows", _p(ex), _DT[ex.dtype], ex.shape[0], h, _p(sc), _p(ofs), groups, per_col,
                  _p(ends), DT_INT64 if ends is not None else DT_NONE, n_e if ends is not None else 0,
                  expert_capacity if (groups > 1 and drop_pad_mode == 1) else 0, _p(y), _stream(ex))
        return y, ri, tok, x.new_empty((0,), dtype=torch.float32)
    _check(offset is None, "npu_moe_init_routing_v2: offset applies to quant_mode 0")
    return _route_v2(x, expert_idx, scale, **route)


_define("npu", "npu_moe_init_routing_v2(Tensor x, Tensor expert_idx, *, Tensor? scale=None, Tensor? offset=None, "
               "int active_num=-1, int expert_capacity=-1, int expert_num=-1, int drop_pad_mode=0, "
               "int expert_tokens_num_type=0, bool expert_tokens_num_flag=False, int quant_mode=-1, "
               "int[] active_expert_range=[], int row_idx_type=0) -> (Tensor, Tensor, Tensor, Tensor)",
        _init_routing_v2_fake, _init_routing_v2_cuda)


# ============================================================================ npu_moe_finalize_routing
def _finalize_dims(expanded, skip1, scales, src_to_dst, expert=None):
    """(tokens, k): from scales [T, k], else expert_for_source_row [T, k], else skip1's T rows."""
    if scales is not None:
        t, k = scales.shape
    elif expert is not None and expert.dim() == 2:
        t, k = expert.shape
    elif skip1 is not None:
        t = skip1.shape[0]
        k = src_to_dst.numel() // max(t, 1)
    else:
        raise RuntimeError("npu_moe_finalize_routing: scales, expert_for_source_row or skip1 is needed to know the "
                           "token count")
    return t, k


def _finalize_fake(expanded_permuted_rows, skip1, skip2, bias, scales, expanded_src_to_dst_row,
                   export_for_source_row, drop_pad_mode=0):
    t, _ = _finalize_dims(expanded_permuted_rows, skip1, scales, expanded_src_to_dst_row, export_for_source_row)
    return expanded_permuted_rows.new_empty((t, expanded_permuted_rows.shape[-1]))


def _finalize_cuda(expanded_permuted_rows, skip1, skip2, bias, scales, expanded_src_to_dst_row,
                   export_for_source_row, drop_pad_mode=0):
    """npu_moe_finalize_routing (npu_moe_finalize_routing.py:21-41)."""
    ex = expanded_permuted_rows
    _on_gpu(ex, skip1, skip2, bias, scales, expanded_src_to_dst_row, export_for_source_row)
    mode = 0 if drop_pad_mode is None else int(drop_pad_mode)
    _check(mode in (0, 2), "npu_moe_finalize_routing: drop_pad_mode must be 0 (k-major slots) or 2 (token-major)")
    t, k = _finalize_dims(ex, skip1, scales, expanded_src_to_dst_row, export_for_source_row)
    h = ex.shape[-1]
    y = ex.new_empty((t, h))
    dt = ex.dtype
    for name, tt in (("skip1", skip1), ("skip2", skip2), ("bias", bias)):
        if tt is not None:
            _check(tt.dtype == dt and tt.shape[-1] == h, f"npu_moe_finalize_routing: {name} must match the rows' dtype/H")
    _check(expanded_src_to_dst_row.dtype == torch.int32 and expanded_src_to_dst_row.numel() == t * k,
           "npu_moe_finalize_routing: expanded_src_to_dst_row must be int32 with T*k entries")
    if bias is not None:
        _check(export_for_source_row is not None, "npu_moe_finalize_routing: bias needs export_for_source_row")
    if t == 0:
        return y
    c = lambda a: None if a is None else a.contiguous()  # noqa: E731
    exc, s1, s2, bi, sc, s2d, efs = map(c, (ex, skip1, skip2, bias, scales, expanded_src_to_dst_row,
                                            export_for_source_row))
    _lib.call("tai_moe_finalize_routing", _p(exc), _DT[dt], t, h, k, _p(s1), _p(s2), _p(bi), _p(sc),
              _DT[sc.dtype] if sc is not None else DT_NONE, _p(s2d), _p(efs), mode, _p(y), _stream(exc))
    return y


_define("npu", "npu_moe_finalize_routing(Tensor expanded_permuted_rows, Tensor? skip1, Tensor? skip2, Tensor? bias, "
               "Tensor? scales, Tensor expanded_src_to_dst_row, Tensor? export_for_source_row, "
               "int? drop_pad_mode=0) -> Tensor", _finalize_fake, _finalize_cuda)


# ============================================================================ fused_infer_attention_score
from . import _fia  # noqa: E402  (attention dispatch lives in its own module)

_FIA_ARGS = ("Tensor query, Tensor key, Tensor value, *, Tensor? pse_shift=None, Tensor? atten_mask=None, "
             "{seq} actual_seq_lengths=None, {seq} actual_seq_lengths_kv=None, Tensor? dequant_scale1=None, "
             "Tensor? quant_scale1=None, Tensor? dequant_scale2=None, Tensor? quant_scale2=None, "
             "Tensor? quant_offset2=None, Tensor? antiquant_scale=None, Tensor? antiquant_offset=None, "
             "{bt_first}"
             "Tensor? key_antiquant_scale=None, Tensor? key_antiquant_offset=None, "
             "Tensor? value_antiquant_scale=None, Tensor? value_antiquant_offset=None, {bt_second}"
             "Tensor? key_shared_prefix=None, Tensor? value_shared_prefix=None, {seq} actual_shared_prefix_len=None, "
             "Tensor? query_rope=None, Tensor? key_rope=None, Tensor? key_rope_antiquant_scale=None, "
             "int num_heads=1, float scale=1.0, int pre_tokens=2147483647, int next_tokens=2147483647, "
             "str input_layout=\"BSH\", int num_key_value_heads=0, int sparse_mode=0, int inner_precise=0, "
             "int block_size=0, int antiquant_mode=0, {tail}) -> (Tensor, Tensor)")
_BT = "Tensor? block_table=None, Tensor? query_padding_size=None, Tensor? kv_padding_size=None, "

# torch_npu order: block_table after antiquant_offset; lse flag before the key/value antiquant modes.
_define("npu", "npu_fused_infer_attention_score(" + _FIA_ARGS.format(
    seq="SymInt[]?", bt_first=_BT, bt_second="",
    tail="bool softmax_lse_flag=False, int key_antiquant_mode=0, int value_antiquant_mode=0"),
    _fia.fia_fake, _fia.fia_cuda)
# air:: (python/torchair/ops/_npu_fused_infer_attention_score.py:14-34): tensor sequence lengths,
# block_table after the value antiquant tensors, lse flag last.
_define("air", "npu_fused_infer_attention_score(" + _FIA_ARGS.format(
    seq="Tensor?", bt_first="", bt_second=_BT,
    tail="int key_antiquant_mode=0, int value_antiquant_mode=0, bool softmax_lse_flag=False"),
    _fia.fia_fake, _fia.fia_cuda)

# npu_fused_infer_attention_score_v2: air:: (python/torchair/ops/_npu_fused_infer_attention_score_v2.py:16-30,
# tensor lengths) and npu:: (torch_npu's op, list lengths, converter .../custom/fused_infer_attention_score_v2.py:14)
_FIA_V2_ARGS = ("Tensor query, Tensor key, Tensor value, *, Tensor? query_rope=None, Tensor? key_rope=None, "
                "Tensor? pse_shift=None, Tensor? atten_mask=None, {seq} actual_seq_qlen=None, "
                "{seq} actual_seq_kvlen=None, Tensor? block_table=None, Tensor? dequant_scale_query=None, "
                "Tensor? dequant_scale_key=None, Tensor? dequant_offset_key=None, Tensor? dequant_scale_value=None, "
                "Tensor? dequant_offset_value=None, Tensor? dequant_scale_key_rope=None, "
                "Tensor? quant_scale_out=None, Tensor? quant_offset_out=None, Tensor? quant_scale_p=None, "
                "Tensor? learnable_sink=None, int num_query_heads=1, int num_key_value_heads=0, "
                "float softmax_scale=1.0, int pre_tokens=2147483647, int next_tokens=2147483647, "
                "str input_layout=\"BSH\", int sparse_mode=0, int block_size=0, int query_quant_mode=0, "
                "int key_quant_mode=0, int value_quant_mode=0, int inner_precise=0, bool return_softmax_lse=False, "
                "int? query_dtype=None, int? key_dtype=None, int? value_dtype=None, int? query_rope_dtype=None, "
                "int? key_rope_dtype=None, int? key_shared_prefix_dtype=None, int? value_shared_prefix_dtype=None, "
                "int? dequant_scale_query_dtype=None, int? dequant_scale_key_dtype=None, "
                "int? dequant_scale_value_dtype=None, int? dequant_scale_key_rope_dtype=None, int? out_dtype=None) "
                "-> (Tensor, Tensor)")
_define("air", "npu_fused_infer_attention_score_v2(" + _FIA_V2_ARGS.format(seq="Tensor?"), _fia.fia_v2_fake,
        _fia.fia_v2_cuda)
_define("npu", "npu_fused_infer_attention_score_v2(" + _FIA_V2_ARGS.format(seq="SymInt[]?"), _fia.fia_v2_fake,
        _fia.fia_v2_cuda)

from . import _norm_cache  # noqa: E402,F401  (RMS-norm family and KV-cache writers)

from . import _gmm_fused  # noqa: E402,F401  (fused MoE grouped GEMMs)
from . import _moe_fused  # noqa: E402,F401  (routing -> grouped GEMM fusion of the compiled graph)
