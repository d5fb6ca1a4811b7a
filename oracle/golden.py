"""CPU oracle for the fused inference ops - TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module,
and only as the checker (or as the timed CPU baseline). The product path never calls it.

The reference ships no arithmetic for these ops: its converters emit opaque GE nodes whose
kernels live in closed CANN packages (python/torchair/_ge_concrete_graph/ge_converter/custom/*.py),
so this module restates each op from its prototype, converter arguments and meta rules
(file:line cited per function). Where those leave a choice open the choice is written here
and frozen by the fixtures in tests/golden/ (written by tests/golden/make_fixtures.py):
  * quantisation: scale = amax/127 (fp32 divide), y = clamp(rint(xs/scale), -128, 127),
    rint = round half to even; an all-zero row gives scale 0 and y 0;
  * dequant_swiglu_quant: d = (float(x [+ int32 bias]) * weight_scale) * activation_scale
    [+ fp32 bias]; activate_left=True -> silu(A)*B else A*silu(B); silu(a) = a/(1+exp(-a));
    group_index holds per-group row COUNTS; rows past the total -> y 0, scale 0;
  * dynamic_quant group_index holds cumulative row ENDS;
  * gating: sigmoid / softmax evaluated in float64 and rounded once to fp32; group score =
    max (mode 0) or top1+top2 (mode 1); ties go to the lower group / expert index; rows are
    ordered by descending score; sigmoid weights are divided by (sequential fp32 sum + eps);
  * routing: slot p = token*k + j, stable sort by expert; finalize drop_pad_mode 0 indexes
    slots k-major (p = j*T + t, legacy routing), 2 token-major (p = t*k + j);
  * attention: padded query rows and empty sequences give zero output and lse = -inf.
All float arithmetic is numpy float32 unless stated (numpy never fuses multiply-add).
Integer GEMMs are exact (float64 products and sums stay below 2**53 for int8 inputs).
"""
from __future__ import annotations

from typing import Optional, Tuple

import numpy as np

F32 = np.float32


# ----------------------------------------------------------------------------- bf16 helpers
def bf16_bits_to_f32(u16: np.ndarray) -> np.ndarray:
    return (np.asarray(u16, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit pattern (NaN kept quiet)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x007FFFFF) != 0)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Rounds fp32 values to the output dtype ('bf16', 'fp16', 'fp32'), returned as fp32."""
    if dtype == "bf16":
        return round_bf16(x)
    if dtype == "fp16":
        return x.astype(np.float16).astype(np.float32)
    return x.astype(np.float32)


# ----------------------------------------------------------------------------- quantisation
def _quant_rows(v: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    amax = np.max(np.abs(v), axis=1) if v.shape[1] else np.zeros(v.shape[0], F32)
    scale = (amax.astype(F32) / F32(127.0)).astype(F32)
    safe = np.where(scale == 0, F32(1.0), scale).astype(F32)
    q = np.rint(v / safe[:, None])
    q = np.where(scale[:, None] == 0, 0, q)
    q = np.clip(q, -128, 127).astype(np.int8)
    return q, scale


def dynamic_quant(x: np.ndarray, smooth_scales: Optional[np.ndarray] = None,
                  group_index: Optional[np.ndarray] = None) -> Tuple[np.ndarray, np.ndarray]:
    """npu_dynamic_quant, symmetric per-token int8.

    Follows python/torchair/_ge_concrete_graph/ge_converter/custom/npu_dynamic_quant.py:8-42
    (pertoken branch -> ge.DynamicQuant) and its prototype
    third_party/ascend/include/ops/op_proto/inc/nn_quantize.h:47-56 (y int8, scale fp32 of
    shape x.shape[:-1]).
    """
    x = np.asarray(x, F32)
    h = x.shape[-1]
    xr = x.reshape(-1, h)
    if smooth_scales is not None:
        sm = np.asarray(smooth_scales, F32)
        if group_index is None:
            xr = (xr * sm.reshape(1, h)).astype(F32)
        else:
            ends = np.asarray(group_index, np.int64)
            g = np.searchsorted(ends, np.arange(xr.shape[0]), side="right")
            g = np.minimum(g, len(ends) - 1)
            xr = (xr * sm.reshape(-1, h)[g]).astype(F32)
    q, s = _quant_rows(xr)
    return q.reshape(x.shape), s.reshape(x.shape[:-1])


def dynamic_quant_v2(x: np.ndarray, smooth_scales: Optional[np.ndarray] = None,
                     group_index: Optional[np.ndarray] = None, symmetric: bool = True, per_tensor: bool = False,
                     dst_type_max: float = 0.0):
    """ge.DynamicQuantV2: npu_dynamic_quant with quant_mode "pertensor" or dst_type_max != 0
    (is_symmetrical=True, .../custom/npu_dynamic_quant.py:21-25) and npu_dynamic_quant_asymmetric
    (is_symmetrical=False, :47-61; prototype nn_quantize.h:77-85). The arithmetic is frozen by this build
    (the reference holds only the prototype): over each row (or the whole input) of the smoothed xs,
    symmetric: scale = max(|max|, |min|) / q (q = dst_type_max or 127), y = clamp(rint(xs / scale));
    asymmetric: hi = max(max, 0), lo = min(min, 0), scale = (hi - lo) / 255, offset = -128 - lo / scale,
    y = clamp(rint(xs / scale + offset)); a zero range gives scale 0, offset 0, y 0. fp32 throughout.
    Returns (y, scale, offset) with offset None when symmetric.
    """
    x = np.asarray(x, F32)
    h = x.shape[-1]
    xr = x.reshape(-1, h)
    if smooth_scales is not None:
        sm = np.asarray(smooth_scales, F32)
        if group_index is None:
            xr = (xr * sm.reshape(1, h)).astype(F32)
        else:
            ends = np.asarray(group_index, np.int64)
            g = np.minimum(np.searchsorted(ends, np.arange(xr.shape[0]), side="right"), len(ends) - 1)
            xr = (xr * sm.reshape(-1, h)[g]).astype(F32)
    stats = xr.reshape(1, -1) if per_tensor else xr
    mx = stats.max(axis=1) if stats.shape[1] else np.zeros(stats.shape[0], F32)
    mn = stats.min(axis=1) if stats.shape[1] else np.zeros(stats.shape[0], F32)
    q = F32(dst_type_max if dst_type_max > 0 else 127.0)
    if symmetric:
        scale = (np.maximum(np.abs(mx), np.abs(mn)).astype(F32) / q).astype(F32)
        offset = np.zeros_like(scale)
    else:
        hi, lo = np.maximum(mx, F32(0)).astype(F32), np.minimum(mn, F32(0)).astype(F32)
        scale = ((hi - lo).astype(F32) / F32(255.0)).astype(F32)
        safe = np.where(scale == 0, F32(1), scale).astype(F32)
        offset = np.where(scale == 0, F32(0), (F32(-128.0) - (lo / safe).astype(F32)).astype(F32)).astype(F32)
    sc_rows = np.broadcast_to(scale, (xr.shape[0],)) if per_tensor else scale
    off_rows = np.broadcast_to(offset, (xr.shape[0],)) if per_tensor else offset
    safe = np.where(sc_rows == 0, F32(1), sc_rows).astype(F32)
    v = (xr / safe[:, None]).astype(F32)
    if not symmetric:
        v = (v + off_rows[:, None]).astype(F32)
    yq = np.where(sc_rows[:, None] == 0, 0, np.clip(np.rint(v), -128, 127)).astype(np.int8)
    shape = (1,) if per_tensor else x.shape[:-1]
    return yq.reshape(x.shape), scale.reshape(shape), (None if symmetric else offset.reshape(shape))


def silu(a: np.ndarray) -> np.ndarray:
    a = np.asarray(a, F32)
    with np.errstate(over="ignore"):  # exp(-a) overflows to inf for a < -88.7, giving silu = -0 as it should
        return (a / (F32(1.0) + np.exp(-a))).astype(F32)


def dequant_swiglu_quant(x: np.ndarray, weight_scale=None, activation_scale=None, bias=None, quant_scale=None,
                         group_index=None, activate_left: bool = False, quant_mode: int = 1,
                         quant_offset=None, swiglu_mode: int = 0, clamp_limit: float = 7.0, glu_alpha: float = 1.702,
                         glu_bias: float = 1.0) -> Tuple[np.ndarray, np.ndarray]:
    """npu_dequant_swiglu_quant, swiglu_mode 0, round_mode 0 (rint). quant_mode 1 (dynamic): per-row
    symmetric int8 of h * quant_scale. quant_mode 0 (static, the converter's default "static",
    npu_dequant_swiglu_quant.py:26-28): y = clamp(rint(h * quant_scale + quant_offset)) with scale 0 (the
    reference holds no kernel fixing it; the formula is the static quantisation rule, pinned by known
    answers).

    Follows .../custom/npu_dequant_swiglu_quant.py:5-47 (round_mode 0 -> "rint", quant_mode 1 ->
    "dynamic"), prototype experiment_ops.h:3765-3812 (activate_left semantics) and the meta rule
    python/torchair/_contrib/custom_torch_ops/auto_register_custom_torch_ops.py:155-191 (last dim
    halved, int8 y, fp32 scale of y.shape[:-1]).
    """
    x = np.asarray(x, np.int32)
    n2 = x.shape[-1]
    n = n2 // 2
    xr = x.reshape(-1, n2)
    rows = xr.shape[0]
    if group_index is not None:
        counts = np.asarray(group_index, np.int64).reshape(-1)
        ends = np.cumsum(counts)
        grp = np.searchsorted(ends, np.arange(rows), side="right")
        live = grp < len(counts)
        grp = np.minimum(grp, len(counts) - 1)
    else:
        grp = np.zeros(rows, np.int64)
        live = np.ones(rows, bool)
    ng = 1 if group_index is None else len(np.asarray(group_index).reshape(-1))
    xi = xr.copy()
    bias_f = None
    if bias is not None:
        b = np.asarray(bias)
        if b.dtype == np.int32:
            xi = (xi + b.reshape(ng, n2)[grp]).astype(np.int32)
        else:
            bias_f = np.asarray(b, F32).reshape(ng, n2)[grp]
    d = xi.astype(F32)
    if weight_scale is not None:
        d = (d * np.asarray(weight_scale, F32).reshape(ng, n2)[grp]).astype(F32)
    if activation_scale is not None:
        d = (d * np.asarray(activation_scale, F32).reshape(rows, 1)).astype(F32)
    if bias_f is not None:
        d = (d + bias_f).astype(F32)
    if swiglu_mode == 1:
        # odd-even blocked columns (prototype experiment_ops.h:3786-3790): output j takes inputs 2j, 2j + 1;
        # the activated one (2j with activate_left) is clamped above at clamp_limit, the other to
        # [-clamp_limit, clamp_limit]; h = g * sigmoid(glu_alpha * g) * (l + glu_bias)
        ev, od = d[:, 0::2], d[:, 1::2]
        lim = F32(clamp_limit)
        g = np.minimum(ev if activate_left else od, lim).astype(F32)
        lin = np.clip(od if activate_left else ev, -lim, lim).astype(F32)
        with np.errstate(over="ignore"):
            sg = (F32(1.0) / (F32(1.0) + np.exp(-(F32(glu_alpha) * g).astype(F32)))).astype(F32)
        r = ((g * sg).astype(F32) * (lin + F32(glu_bias)).astype(F32)).astype(F32)
    else:
        a, b2 = d[:, :n], d[:, n:]
        r = (silu(a) * b2).astype(F32) if activate_left else (a * silu(b2)).astype(F32)
    if quant_scale is not None:
        r = (r * np.asarray(quant_scale, F32).reshape(ng, n)[grp]).astype(F32)
    if quant_mode == 0:
        of = np.zeros((ng, n), F32) if quant_offset is None else np.asarray(quant_offset, F32).reshape(ng, n)
        q = np.clip(np.rint((r + of[grp]).astype(F32)), -128, 127).astype(np.int8)
        s = np.zeros(rows, F32)
    else:
        q, s = _quant_rows(r)
    q[~live] = 0
    s[~live] = 0
    return q.reshape(x.shape[:-1] + (n,)), s.reshape(x.shape[:-1])


# ----------------------------------------------------------------------------- int8 GEMMs
def int_matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Exact int8 x int8 -> int64 product (float64 BLAS; |partial sums| < 2**53)."""
    return np.rint(np.asarray(a, np.float64) @ np.asarray(b, np.float64)).astype(np.int64)


def _epilogue(acc: np.ndarray, scale, pts, bias, out_dtype: str, col_scale_rows=None) -> np.ndarray:
    acc32 = acc.astype(np.int64)
    bias_f = None
    if bias is not None:
        bb = np.asarray(bias)
        if bb.dtype == np.int32:
            acc32 = acc32 + bb.astype(np.int64)
        else:
            bias_f = np.asarray(bb, F32)
    acc32 = ((acc32 + 2 ** 31) % 2 ** 32 - 2 ** 31).astype(np.int32)  # int32 wrap-around
    if out_dtype == "int32":
        return acc32
    v = acc32.astype(F32)
    if scale is not None:
        v = (v * np.asarray(scale, F32)).astype(F32)
    if pts is not None:
        v = (v * np.asarray(pts, F32).reshape(-1, 1)).astype(F32)
    if bias_f is not None:
        v = (v + bias_f).astype(F32)
    return round_to(v, out_dtype)


def quant_matmul(x1, x2, scale=None, pertoken_scale=None, bias=None, out_dtype: str = "bf16",
                 offset=None) -> np.ndarray:
    """npu_quant_matmul W8A8: exact int32 accumulation, then (acc [+int32 bias]) * scale[n] * pertoken[m]
    [+ fp32 bias], rounded to out_dtype.

    Follows .../custom/quantmatmul.py:63-255 (x2 is [K, N]: trans_x2 = x1[-1] == x2[-2] at :129;
    ge.QuantBatchMatmulV3(x1, x2, scale, offset, bias, pertoken_scale, dtype) at :244-254) and
    the dtype table of fusion_ops.h:380-451.
    """
    acc = int_matmul(x1, x2)
    sc = None if scale is None else np.asarray(scale, F32).reshape(1, -1)
    if out_dtype == "int8":
        # the converter's default output (output_dtype None -> 1, quantmatmul.py:91-92): fp32
        # (acc [+ int32 bias]) * scale [* pertoken] [+ offset], then round half to even and saturate
        v = _epilogue(acc, sc, pertoken_scale, bias, "fp32")
        if offset is not None:
            v = (v + np.asarray(offset, F32).reshape(1, -1)).astype(F32)
        return np.clip(np.rint(v), -128, 127).astype(np.int8)
    return _epilogue(acc, sc, pertoken_scale, bias, out_dtype)


def group_offsets(group_list, list_type: int, m: int) -> Tuple[np.ndarray, np.ndarray]:
    gl = np.asarray(group_list, np.int64).reshape(-1)
    if list_type == 1:
        ends = np.cumsum(np.maximum(gl, 0))
    else:
        ends = np.maximum.accumulate(gl)
    begins = np.concatenate([[0], ends[:-1]])
    return np.minimum(begins, m), np.minimum(ends, m)


def grouped_matmul(x, w, group_list, group_list_type: int = 0, scale=None, per_token_scale=None, bias=None,
                   out_dtype: str = "int32") -> np.ndarray:
    """npu_grouped_matmul int8 path, split_item 2/3, group_type 0: rows [off_e, off_e+1) use w[e].

    Follows .../custom/grouped_matmul.py:210-365 (int8 bias filled as int32 :252-258; output_dtype
    -> y_dtype table convert_ydtype_in_a8 :178-195) and prototype experiment_ops.h:3636-3662.
    group_list_type 0 = cumulative ends, 1 = counts. Rows past the last group are zero.
    """
    x = np.asarray(x)
    w = np.asarray(w)
    m = x.shape[0]
    e_cnt, _, n = w.shape
    out = np.zeros((m, n), np.int32 if out_dtype == "int32" else F32)
    b, en = group_offsets(group_list, group_list_type, m)
    for e in range(e_cnt):
        if en[e] <= b[e]:
            continue
        acc = int_matmul(x[b[e]:en[e]], w[e])
        sc = None if scale is None else np.asarray(scale, F32).reshape(e_cnt, n)[e].reshape(1, n)
        pts = None if per_token_scale is None else np.asarray(per_token_scale, F32)[b[e]:en[e]]
        bi = None if bias is None else np.asarray(bias).reshape(e_cnt, n)[e].reshape(1, n)
        out[b[e]:en[e]] = _epilogue(acc, sc, pts, bi, out_dtype)
    return out


# ----------------------------------------------------------------------------- MoE gating / routing
def moe_gating_top_k(x, k: int, bias=None, k_group: int = 1, group_count: int = 1, group_select_mode: int = 0,
                     renorm: int = 0, norm_type: int = 0, out_flag: bool = False,
                     routed_scaling_factor: float = 1.0, eps: float = 1e-20, out_dtype: str = "fp32"):
    """npu_moe_gating_top_k (DeepSeek-V3 grouped "noaux_tc" selection).

    Follows .../custom/npu_moe_gating_top_k.py:4-22 (attributes passed to ge.MoeGatingTopK),
    prototype experiment_ops.h:3723-3764, meta auto_register_custom_torch_ops.py:103-114
    (y [T,k] of x dtype, expert_idx int32 [T,k], out fp32 [T,E]).
    Returns (y, expert_idx, out).
    """
    if renorm != 0:
        raise NotImplementedError("renorm must be 0")
    x = np.asarray(x, F32)
    t, e = x.shape
    x64 = x.astype(np.float64)
    if norm_type == 1:
        s = (1.0 / (1.0 + np.exp(-x64))).astype(F32)
    else:
        m = np.max(x, axis=1, keepdims=True).astype(np.float64)
        ex = np.exp(x64 - m)
        s = (ex / np.sum(ex, axis=1, keepdims=True)).astype(F32)
    sb = s if bias is None else (s + np.asarray(bias, F32).reshape(1, e)).astype(F32)
    sb = sb.copy()
    if group_count > 1:
        gsz = e // group_count
        g = sb.reshape(t, group_count, gsz)
        if group_select_mode == 1 and gsz > 1:
            srt = -np.sort(-g, axis=2)
            gs = (srt[:, :, 0] + srt[:, :, 1]).astype(F32)
        else:
            gs = np.max(g, axis=2)
        order = np.argsort(-gs, axis=1, kind="stable")
        keep = np.zeros((t, group_count), bool)
        np.put_along_axis(keep, order[:, :k_group], True, axis=1)
        sb[~np.repeat(keep, gsz, axis=1)] = -np.inf
    idx = np.argsort(-sb, axis=1, kind="stable")[:, :k].astype(np.int32)
    w = np.take_along_axis(s, idx.astype(np.int64), axis=1).astype(F32)
    if norm_type == 1:
        tot = np.zeros(t, F32)
        for j in range(k):
            tot = (tot + w[:, j]).astype(F32)
        w = (w / (tot + F32(eps))[:, None]).astype(F32)
    w = (w * F32(routed_scaling_factor)).astype(F32)
    return round_to(w, out_dtype), idx, s


def moe_init_routing_v2(x, expert_idx, scale=None, active_rows: Optional[int] = None, expert_start: int = 0,
                        expert_end: Optional[int] = None, expert_tokens_num_type: int = 0, row_idx_type: int = 0):
    """npu_moe_init_routing_v2, dropless (drop_pad_mode 0), quant_mode -1. (quant_mode 1 without smooth
    scales is this followed by dynamic_quant of the expanded rows; the tests compose the two.)

    Follows .../custom/npu_moe_init_routing_v2.py:41-91 (-> ge.MoeInitRoutingV3) and prototype
    experiment_ops.h:2138-2190 (row_idx_type 0 gather / 1 scatter, expert_tokens_num_type 0
    cumsum / 1 count, active_expert_range). Returns
    (expanded_x, expanded_row_idx, expert_tokens, expanded_scale_or_None).
    """
    x = np.asarray(x)
    ei = np.asarray(expert_idx, np.int64)
    t, k = ei.shape
    n = t * k
    if expert_end is None:
        expert_end = int(ei.max()) + 1 if n else 1
    rows = n if active_rows is None else active_rows
    flat = ei.reshape(-1)
    valid = (flat >= expert_start) & (flat < expert_end)
    slots = np.nonzero(valid)[0]
    order = slots[np.argsort(flat[slots], kind="stable")]
    total = len(order)
    ex = np.zeros((rows,) + x.shape[1:], x.dtype)
    live = min(rows, total)
    ex[:live] = x[order[:live] // k]
    ri = np.full(n, -1, np.int32)
    if row_idx_type == 0:
        ri[order] = np.arange(total, dtype=np.int32)
    else:
        ri[:total] = order.astype(np.int32)
    counts = np.bincount(flat[valid] - expert_start, minlength=expert_end - expert_start).astype(np.int64)
    tokens = np.cumsum(counts) if expert_tokens_num_type == 0 else counts
    es = None
    if scale is not None:
        es = np.zeros(rows, F32)
        es[:live] = np.asarray(scale, F32)[order[:live] // k]
    return ex, ri, tokens, es


def moe_init_routing_v2_droppad(x, expert_idx, capacity: int, scale=None, expert_start: int = 0,
                                expert_end: Optional[int] = None, expert_tokens_num_type: int = 0):
    """npu_moe_init_routing_v2 with drop_pad_mode 1 and expert_capacity (prototype
    experiment_ops.h:2160-2189: drop_pad_mode 1 = dropPad, expert_capacity = the max tokens of every
    expert; converter .../custom/npu_moe_init_routing_v2.py:41-91). Expert e (of the range) owns rows
    [e * capacity, (e + 1) * capacity) of expanded_x; its slots, in the dropless order (stable by slot
    t * k + j), fill them and slots past the capacity are dropped (row index -1); unfilled rows are
    zero. expert_tokens counts every slot routed to the expert (cumsum for type 0). Returns
    (expanded_x [E * capacity, H], expanded_row_idx [T * k], expert_tokens, expanded_scale_or_None).
    The reference holds no kernel or test for this mode; the layout is pinned against the dropless
    routing (capacity >= the largest expert count gives its rows, placed at each expert's block).
    """
    x = np.asarray(x)
    ei = np.asarray(expert_idx, np.int64)
    t, k = ei.shape
    n = t * k
    if expert_end is None:
        expert_end = int(ei.max()) + 1 if n else 1
    bins = expert_end - expert_start
    flat = ei.reshape(-1)
    ex = np.zeros((bins * capacity,) + x.shape[1:], x.dtype)
    ri = np.full(n, -1, np.int32)
    es = None if scale is None else np.zeros(bins * capacity, F32)
    fill = np.zeros(bins, np.int64)
    for p in range(n):  # slots in order: the stable per-expert order
        e = int(flat[p]) - expert_start
        if e < 0 or e >= bins:
            continue
        if fill[e] < capacity:
            q = e * capacity + fill[e]
            ri[p] = q
            ex[q] = x[p // k]
            if es is not None:
                es[q] = np.asarray(scale, F32)[p // k]
        fill[e] += 1
    counts = fill.astype(np.int64)
    tokens = np.cumsum(counts) if expert_tokens_num_type == 0 else counts
    return ex, ri, tokens, es


def static_quant_rows(x, scale, offset=None, group_of_row=None):
    """quant_mode 0 (static) of npu_moe_init_routing_v2 (prototype experiment_ops.h:2160-2189; the scale and
    offset inputs of MoeInitRoutingV3 :2140-2158, offset [experts, 1] or [experts, H]):
    y = clamp(rint(x * scale + offset), -128, 127) in fp32, each operation rounded once. scale / offset
    are [1], [G, 1] or [G, H] (G groups, a row taking group_of_row[row]) or [1, H]; offset None is 0.
    The reference holds no kernel for it; pinned by known answers (round half to even, saturation).
    """
    x = np.asarray(x, F32)
    rows, h = x.shape
    sc = np.asarray(scale, F32)
    of = np.zeros_like(sc) if offset is None else np.asarray(offset, F32)
    sc2 = sc.reshape(-1, 1) if sc.ndim <= 1 or sc.shape[-1] == 1 else sc.reshape(-1, h)
    of2 = of.reshape(sc2.shape)
    g = np.zeros(rows, np.int64) if group_of_row is None or sc2.shape[0] == 1 else np.asarray(group_of_row, np.int64)
    y = (x * sc2[g]).astype(F32) + of2[g]
    return np.clip(np.rint(y.astype(F32)), -128, 127).astype(np.int8)


def moe_init_routing(x, row_idx, expert_idx, active_num: int):
    """npu_moe_init_routing (legacy). Follows .../custom/moe_init_routing.py:4-21 and prototype
    experiment_ops.h:2112-2135. Returns (expanded_x, expanded_row_idx, expanded_expert_idx)."""
    x = np.asarray(x)
    ri = np.asarray(row_idx, np.int64).reshape(-1)
    ei = np.asarray(expert_idx, np.int64)
    t, k = ei.shape
    flat = ei.reshape(-1)
    order = np.argsort(flat, kind="stable")
    n = t * k
    rows = min(t, active_num) * k if active_num >= 0 else n
    ex = x[ri[order[:rows]] % t]
    eri = np.zeros(n, np.int32)
    eri[ri[order]] = np.arange(n, dtype=np.int32)
    eei = flat[order].astype(np.int32)
    return ex, eri, eei


def moe_finalize_routing(expanded, skip1, skip2, bias, scales, src_to_dst, expert_for_source_row,
                         drop_pad_mode: int = 0, out_dtype: str = "bf16") -> np.ndarray:
    """npu_moe_finalize_routing: y[t] = skip1 + skip2 + sum_j scales[t,j]*(expanded[src_to_dst[p]] + bias[expert]).

    Follows .../custom/npu_moe_finalize_routing.py:4-41 (declared cases: arange row index, optional
    skip2/bias/scales) and prototype experiment_ops.h:2196-2219. fp32 accumulation in the order
    skip1, skip2, j = 0..k-1.
    """
    ex = np.asarray(expanded, F32)
    s2d = np.asarray(src_to_dst, np.int64).reshape(-1)
    if scales is not None:
        t, k = np.asarray(scales).shape
    elif expert_for_source_row is not None:
        t, k = np.asarray(expert_for_source_row).shape
    else:
        t = np.asarray(skip1).shape[0]
        k = len(s2d) // t
    h = ex.shape[-1]
    acc = np.zeros((t, h), F32)
    if skip1 is not None:
        acc = np.asarray(skip1, F32).copy()
    if skip2 is not None:
        acc = (acc + np.asarray(skip2, F32)).astype(F32)
    tt = np.arange(t)
    for j in range(k):
        p = j * t + tt if drop_pad_mode == 0 else tt * k + j
        d = s2d[p]
        ok = d >= 0
        v = np.zeros((t, h), F32)
        v[ok] = ex[d[ok]]
        if bias is not None:
            e = np.asarray(expert_for_source_row, np.int64).reshape(t, k)[:, j]
            v = (v + np.asarray(bias, F32)[e]).astype(F32)
        w = np.ones(t, F32) if scales is None else np.asarray(scales, F32)[:, j]
        contrib = (w[:, None] * v).astype(F32)
        acc = np.where(ok[:, None], (acc + contrib).astype(F32), acc)
    return round_to(acc, out_dtype)


# ----------------------------------------------------------------------------- attention
def _softmax_attend(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, mask: Optional[np.ndarray] = None,
                    bias: Optional[np.ndarray] = None, sink: Optional[float] = None):
    """q [n, d], k [L, d], v [L, dv] -> (out [n, dv], lse [n]); fp32, masked entries excluded; bias [n, L]
    (pse_shift) is added to the scaled scores; sink (learnable_sink, one logit) joins the softmax's
    denominator and contributes no value: softmax over [scores, sink] with the sink's column dropped."""
    s = (q.astype(F32) @ k.astype(F32).T) * F32(scale)
    if bias is not None:
        s = (s + np.asarray(bias, F32)).astype(F32)
    if mask is not None:
        s = np.where(mask, s, -np.inf)
    m = np.max(s, axis=1, keepdims=True) if s.shape[1] else np.full((s.shape[0], 1), -np.inf, F32)
    if sink is not None:
        m = np.maximum(m, F32(sink))
    m_safe = np.where(np.isfinite(m), m, 0).astype(F32)
    p = np.exp(s - m_safe)
    den = np.sum(p, axis=1, keepdims=True)
    if sink is not None:
        den = (den + np.exp(F32(sink) - m_safe)).astype(F32)
    with np.errstate(invalid="ignore", divide="ignore"):
        o = np.where(den > 0, (p @ v.astype(F32)) / np.where(den > 0, den, 1), 0).astype(F32)
        lse = np.where(den[:, 0] > 0, m_safe[:, 0] + np.log(np.where(den[:, 0] > 0, den[:, 0], 1)), -np.inf)
    return o, lse.astype(F32)


def paged_decode_attention(q, k_cache, v_cache, block_table, seq_lens, scale: float):
    """npu_fused_infer_attention_score, paged decode (one query token, GQA).

    Follows .../custom/fused_infer_attention_score.py:4-109 (block_table / block_size /
    actual_seq_lengths_kv / num_key_value_heads arguments), prototype experiment_ops.h:3878-3965
    and the output rules of python/torchair/ops/_npu_fused_infer_attention_score.py:160-374.
    q [B, Hq, D]; caches [blocks, bs, Hkv, D]; token t of sequence b lives at
    cache[block_table[b, t // bs], t % bs]. Returns (out [B,Hq,D] fp32, lse [B,Hq]).
    """
    q = np.asarray(q, F32)
    b_cnt, hq, d = q.shape
    _, bs, hkv, _ = k_cache.shape
    g = hq // hkv
    out = np.zeros((b_cnt, hq, d), F32)
    lse = np.full((b_cnt, hq), -np.inf, F32)
    for b in range(b_cnt):
        L = int(seq_lens[b])
        if L <= 0:
            continue
        pages = np.asarray(block_table[b][: (L + bs - 1) // bs], np.int64)
        kk = np.asarray(k_cache[pages], F32).reshape(-1, hkv, d)[:L]
        vv = np.asarray(v_cache[pages], F32).reshape(-1, hkv, d)[:L]
        for h in range(hkv):
            o, l = _softmax_attend(q[b, h * g:(h + 1) * g], kk[:, h], vv[:, h], scale)
            out[b, h * g:(h + 1) * g] = o
            lse[b, h * g:(h + 1) * g] = l
    return out, lse


def band_mask(lq: int, lk: int, origin: int, pre: int, nxt: int) -> np.ndarray:
    """Visibility of kv j (of lk) to query i (of lq): -pre <= j - i - off <= nxt, with off = lk - lq for
    origin 1 (bottom-right) and 0 for origin 0 (top-left); pre / nxt >= 2**31 - 1 are no bound.

    The sparse_mode / pre_tokens / next_tokens attributes of FusedInferAttentionScore (prototype
    experiment_ops.h:3878-3965; converter .../custom/fused_infer_attention_score.py:36-40, 105-106):
    mode 2 = (0, inf, 0), mode 3 = (1, inf, 0), mode 0 = (0, pre, next), mode 4 = (1, pre, next).
    """
    big = 2147483647
    off = (lk - lq) if origin == 1 else 0
    rel = np.arange(lk)[None, :] - np.arange(lq)[:, None] - off
    ok = np.ones((lq, lk), bool)
    if pre < big:
        ok &= rel >= -pre
    if nxt < big:
        ok &= rel <= nxt
    return ok


def prefill_attention(q, k, v, seq_q, seq_kv, causal: int, scale: float, band=None, mask=None, pse=None, sink=None):
    """npu_fused_infer_attention_score, dense prefill. q [B,Sq,Hq,D], k/v [B,Skv,Hkv,D].

    causal 1 (sparse_mode 3, right-down): query i sees kv j <= i + (Lkv - Lq); causal 2
    (sparse_mode 2, left-up): j <= i; 0: no mask. band = (origin, pre, next) replaces causal with
    band_mask's rule. mask: an explicit atten_mask [B or 1, Sq, Skv] (nonzero = masked out, the
    converter's atten_mask input, .../custom/fused_infer_attention_score.py:4-109), combined with the
    rest. pse: pse_shift [B or 1, Hq, >= Sq, >= Skv], added to the scaled scores before the softmax,
    softmax(scale * q.k + pse) (the converter passes pse_type 0, .../custom/fused_infer_attention_score.py:
    94-109; the formula is the one of the public operator documentation, unpinned by the reference beyond
    the reduction pse = 0 -> no pse). sink: learnable_sink [Hq] (one logit per query head in the scaled-score
    domain, _softmax_attend's rule). Rows at or past Lq are zero.
    Returns (out fp32 [B,Sq,Hq,D], lse [B,Hq,Sq]).
    """
    q = np.asarray(q, F32)
    b_cnt, sq, hq, d = q.shape
    skv, hkv = k.shape[1], k.shape[2]
    g = hq // hkv
    out = np.zeros_like(q)
    lse = np.full((b_cnt, hq, sq), -np.inf, F32)
    for b in range(b_cnt):
        lq = sq if seq_q is None else int(seq_q[b])
        lk = skv if seq_kv is None else int(seq_kv[b])
        ii = np.arange(lq)[:, None]
        jj = np.arange(lk)[None, :]
        vis = None
        if band is not None:
            vis = band_mask(lq, lk, *band)
        elif causal == 1:
            vis = jj <= ii + (lk - lq)
        elif causal == 2:
            vis = jj <= ii
        if mask is not None:
            mb = np.asarray(mask)
            mb = mb[0 if mb.shape[0] == 1 else b, :lq, :lk] == 0
            vis = mb if vis is None else (vis & mb)
        for h in range(hq):
            bias = None
            if pse is not None:
                pb = np.asarray(pse, F32)
                bias = pb[0 if pb.shape[0] == 1 else b, h, :lq, :lk]
            o, l = _softmax_attend(q[b, :lq, h], np.asarray(k[b, :lk, h // g], F32),
                                   np.asarray(v[b, :lk, h // g], F32), scale, vis, bias,
                                   None if sink is None else float(np.asarray(sink, F32)[h]))
            out[b, :lq, h] = o
            lse[b, h, :lq] = l
    return out, lse


def paged_prefill_attention(q, k_cache, v_cache, block_table, seq_q, seq_kv, band, scale: float, mask=None,
                            pse=None, sink=None):
    """npu_fused_infer_attention_score with a block table and several query tokens per sequence
    (chunked prefill / multi-token decode). q [B,Sq,Hq,D]; caches [blocks, bs, Hkv, D]; token t of
    sequence b at cache[block_table[b, t // bs], t % bs] (the paged rule of paged_decode_attention);
    band = (origin, pre, next) as in band_mask. Returns (out fp32 [B,Sq,Hq,D], lse [B,Hq,Sq]).
    """
    b_cnt = q.shape[0]
    bs, hkv, d = k_cache.shape[1], k_cache.shape[2], k_cache.shape[3]
    lmax = max(int(x) for x in seq_kv) if b_cnt else 0
    k = np.zeros((b_cnt, lmax, hkv, d), F32)
    v = np.zeros((b_cnt, lmax, hkv, d), F32)
    for b in range(b_cnt):
        L = int(seq_kv[b])
        pages = np.asarray(block_table[b][: (L + bs - 1) // bs], np.int64)
        k[b, :L] = np.asarray(k_cache[pages], F32).reshape(-1, hkv, d)[:L]
        v[b, :L] = np.asarray(v_cache[pages], F32).reshape(-1, hkv, d)[:L]
    return prefill_attention(q, k, v, seq_q, seq_kv, 0, scale, band=band, mask=mask, pse=pse, sink=sink)


def cum_to_lens(cum) -> np.ndarray:
    """Per-sequence lengths of cumulative ends (the TND actual_seq_lengths convention)."""
    c = np.concatenate([[0], np.asarray(cum, np.int64)])
    return np.diff(c)


def unpack_tnd(x, cum, smax: int):
    """Packed rows [T, N, D] (TND; sequence b holds rows [cum[b-1], cum[b])) -> [B, smax, N, D], the rows
    past each sequence's length zero. The TND / NTD query layouts of npu_fused_infer_attention_score
    (python/torchair/ops/_npu_fused_infer_attention_score.py:171-180, 227-239, 300-327)."""
    x = np.asarray(x)
    lens = cum_to_lens(cum)
    out = np.zeros((len(lens), smax) + x.shape[1:], x.dtype)
    start = 0
    for b, ln in enumerate(lens):
        out[b, :ln] = x[start:start + ln]
        start += ln
    return out


def pack_tnd(x, lens):
    """The inverse of unpack_tnd: [B, S, N, D] with per-sequence lengths -> [sum(lens), N, D]."""
    x = np.asarray(x)
    return np.concatenate([x[b, :int(ln)] for b, ln in enumerate(lens)], axis=0)


def packed_prefill_attention(q, k, v, cum_q, cum_kv, causal: int, scale: float, band=None, mask=None, sink=None):
    """npu_fused_infer_attention_score with packed TND queries, keys and values: q [Tq, Hq, D], k/v
    [Tkv, Hkv, D]; actual_seq_lengths / actual_seq_lengths_kv are cumulative ends (torch_npu's TND
    convention; the reference fixes only the TND shapes, _npu_fused_infer_attention_score.py:227-239 and
    the lse [T, N, 1] of :319-327). Each sequence is attended as prefill_attention attends a batch row.
    Returns (out fp32 [Tq, Hq, Dv], lse [Tq, Hq]); rows past the last end are zero (lse -inf)."""
    lq, lk = cum_to_lens(cum_q), cum_to_lens(cum_kv)
    sq, skv = max(int(lq.max(initial=0)), 1), max(int(lk.max(initial=0)), 1)
    o, l = prefill_attention(unpack_tnd(q, cum_q, sq), unpack_tnd(k, cum_kv, skv), unpack_tnd(v, cum_kv, skv),
                             lq, lk, causal, scale, band=band, mask=mask, sink=sink)
    tq = np.asarray(q).shape[0]
    out = np.zeros((tq,) + o.shape[2:], F32)
    lse = np.full((tq, o.shape[2]), -np.inf, F32)
    n = int(lq.sum())
    out[:n] = pack_tnd(o, lq)
    lse[:n] = pack_tnd(np.transpose(l, (0, 2, 1)), lq)
    return out, lse


def with_shared_prefix(k, v, seq_kv, k_prefix, v_prefix, prefix_len: int):
    """Shared prefix of npu_fused_infer_attention_score (key_shared_prefix / value_shared_prefix /
    actual_shared_prefix_len, prototype experiment_ops.h:3933-3935, passed on by the converter,
    .../custom/fused_infer_attention_score.py:29-31, 94-109): the first prefix_len rows of the
    [Sp, Hkv, D] prefix precede every sequence's own keys and values. k/v [B, Skv, Hkv, D]; returns
    (k', v' [B, prefix_len + Skv, Hkv, D], seq_kv' [B]) for prefill_attention, whose atten_mask,
    pse_shift and causal offsets then index the concatenated positions."""
    k, v = np.asarray(k, F32), np.asarray(v, F32)
    b_cnt, skv = k.shape[0], k.shape[1]
    lp = int(prefix_len)
    lens = [skv if seq_kv is None else int(seq_kv[b]) for b in range(b_cnt)]
    kk = np.zeros((b_cnt, lp + skv) + k.shape[2:], F32)
    vv = np.zeros((b_cnt, lp + skv) + v.shape[2:], F32)
    for b in range(b_cnt):
        kk[b, :lp] = np.asarray(k_prefix, F32)[:lp]
        vv[b, :lp] = np.asarray(v_prefix, F32)[:lp]
        kk[b, lp:lp + lens[b]] = k[b, :lens[b]]
        vv[b, lp:lp + lens[b]] = v[b, :lens[b]]
    return kk, vv, np.asarray([lp + x for x in lens], np.int64)


def antiquant_kv(x, scale, offset=None, mode: int = 0):
    """Dequantisation of an int8 key / value of npu_fused_infer_attention_score:
    (x + offset) * scale in fp32. x is [B, S, Hkv, D] (dense, or gathered from a paged cache in
    sequence order); mode 0 (per channel): scale / offset hold Hkv * D values; mode 1 (per token):
    scale / offset are [B, S'] with S' >= S, token t of sequence b taking entry (b, t).

    The inputs are the antiquant tensors of the prototype (experiment_ops.h:3922-3932:
    antiquant_scale / antiquant_offset, key_/value_antiquant_scale / _offset with antiquant_mode,
    key_/value_antiquant_mode), passed on unchanged by the converter
    (.../custom/fused_infer_attention_score.py:16-27). The formula is the antiquant rule
    (x + offset) * scale; the reference holds no kernel that fixes its rounding, so it is pinned here by
    reduction (scale 1 and offset 0 give the integer values themselves; per-channel and per-token
    scales of one value equal each other).
    """
    x = np.asarray(x, F32)
    b_cnt, s_len, hkv, d = x.shape
    sc = np.asarray(scale, F32)
    of = np.zeros_like(sc) if offset is None else np.asarray(offset, F32)
    if mode == 0:
        sc = sc.reshape(1, 1, hkv, d)
        of = of.reshape(1, 1, hkv, d)
    else:
        sc = sc.reshape(b_cnt, -1)[:, :s_len].reshape(b_cnt, s_len, 1, 1)
        of = of.reshape(b_cnt, -1)[:, :s_len].reshape(b_cnt, s_len, 1, 1)
    return ((x + of) * sc).astype(F32)


def quant_attention_out(out, scale2, offset2=None):
    """int8 attention_out of npu_fused_infer_attention_score with quant_scale2 / quant_offset2
    (experiment_ops.h:3943; prototype inputs :3925-3926): clamp(rint(o * scale + offset), -128, 127) in
    fp32, round half to even. out is [B, S, Hq, D] fp32; scale / offset hold 1 value (per tensor) or
    Hq * D values (channel h * D + d)."""
    out = np.asarray(out, F32)
    hq, d = out.shape[2], out.shape[3]
    sc = np.asarray(scale2, F32).reshape(-1)
    of = np.zeros_like(sc) if offset2 is None else np.asarray(offset2, F32).reshape(-1)
    if sc.size != 1:
        sc = sc.reshape(hq, d)
        of = of.reshape(hq, d)
    y = (out * sc).astype(F32) + of
    return np.clip(np.rint(y.astype(F32)), -128, 127).astype(np.int8)


def quant_query_attention(q, k, v, dequant_scale1: float, quant_scale1: float, dequant_scale2: float, seq_q, seq_kv,
                          band, scale: float, mask=None):
    """npu_fused_infer_attention_score with an int8 query, key and value (dequant_scale1, quant_scale1,
    dequant_scale2; prototype experiment_ops.h:3878-3912 types them UINT64 / fp32 / UINT64, an fp32 in
    the low 32 bits of each UINT64; the reference fixes no formula, so this convention is parity
    unpinned beyond the checks of its tests):
      S = (float(int32 q.k) * dequant_scale1) * scale over the visible keys (band / mask as in
          prefill_attention), m = max S, l = sum exp(S - m) in fp32;
      P8 = clamp(rint(exp(S - m) * quant_scale1), 0, 127) (int8, the query-side quantisation of P);
      O = (float(int32 P8.V) * dequant_scale2) / l.
    q [B, Sq, Hq, D], k/v [B, Skv, Hkv, D] int8; returns (out fp32 [B, Sq, Hq, D], lse [B, Hq, Sq] of S)."""
    q, k, v = (np.asarray(t, np.int64) for t in (q, k, v))
    b_cnt, sq, hq, d = q.shape
    skv, hkv, dv = k.shape[1], k.shape[2], v.shape[3]
    g = hq // hkv
    out = np.zeros((b_cnt, sq, hq, dv), F32)
    lse = np.full((b_cnt, hq, sq), -np.inf, F32)
    for bi in range(b_cnt):
        lq = sq if seq_q is None else int(seq_q[bi])
        lk = skv if seq_kv is None else int(seq_kv[bi])
        vis = band_mask(lq, lk, *band)
        if mask is not None:
            mb = np.asarray(mask)
            vis = vis & (mb[0 if mb.shape[0] == 1 else bi, :lq, :lk] == 0)
        for h in range(hq):
            dot = q[bi, :lq, h] @ k[bi, :lk, h // g].T                      # exact int32 values
            s = ((dot.astype(F32) * F32(dequant_scale1)).astype(F32) * F32(scale)).astype(F32)
            s = np.where(vis, s, -np.inf)
            m = s.max(axis=1, keepdims=True) if lk else np.full((lq, 1), -np.inf, F32)
            live = np.isfinite(m[:, 0])
            ms = np.where(np.isfinite(m), m, 0).astype(F32)
            p = np.where(vis, np.exp((s - ms).astype(F32)), 0).astype(F32)
            l = p.sum(axis=1, dtype=F32)
            p8 = np.clip(np.rint((p * F32(quant_scale1)).astype(F32)), 0, 127).astype(np.int64)
            acc = p8 @ v[bi, :lk, h // g]                                   # exact int32 values
            o = (acc.astype(F32) * F32(dequant_scale2)).astype(F32)
            with np.errstate(invalid="ignore", divide="ignore"):
                o = np.where(live[:, None] & (l[:, None] > 0), o / np.where(l > 0, l, 1)[:, None], 0).astype(F32)
                lse[bi, h, :lq] = np.where(live, ms[:, 0] + np.log(np.where(l > 0, l, 1)), -np.inf)
            out[bi, :lq, h] = o
    return out, lse


def mla_decode_attention(q_nope, q_rope, ckv, ckv_scale, krope, block_table, seq_lens, scale: float):
    """npu_fused_infer_attention_score, MLA absorbed decode with an int8 latent cache.

    Follows the query_rope / key_rope / key_antiquant_scale / key_antiquant_mode arguments of
    .../custom/fused_infer_attention_score.py:4-109 and get_value_d in
    python/torchair/ops/_npu_fused_infer_attention_score.py:242-264 (output head dim = latent dim).
    Latent c[t] = int8[t] * scale[t] serves as key (with k_rope appended) and value.
    q_nope [B,H,Dn], q_rope [B,H,Dr], ckv [blocks,bs,Dn] int8, ckv_scale [blocks,bs], krope [blocks,bs,Dr].
    """
    qn = np.asarray(q_nope, F32)
    qr = np.asarray(q_rope, F32)
    b_cnt, h, dn = qn.shape
    bs = ckv.shape[1]
    out = np.zeros((b_cnt, h, dn), F32)
    lse = np.full((b_cnt, h), -np.inf, F32)
    for b in range(b_cnt):
        L = int(seq_lens[b])
        if L <= 0:
            continue
        pages = np.asarray(block_table[b][: (L + bs - 1) // bs], np.int64)
        c = (np.asarray(ckv[pages], F32).reshape(-1, dn)[:L] *
             np.asarray(ckv_scale[pages], F32).reshape(-1)[:L, None]).astype(F32)
        kr = np.asarray(krope[pages], F32).reshape(-1, krope.shape[-1])[:L]
        qk = np.concatenate([qn[b], qr[b]], axis=1)
        kk = np.concatenate([c, kr], axis=1)
        o, l = _softmax_attend(qk, kk, c, scale)
        out[b] = o
        lse[b] = l
    return out, lse


def mla_attention(q_nope, q_rope, ckv, ckv_scale, krope, block_table, seq_q, seq_kv, band, scale: float, sink=None):
    """MLA over a paged latent cache with several query tokens per sequence (MTP / speculative
    decode): the arguments of mla_decode_attention with q_nope [B,Sq,H,Dn], q_rope [B,Sq,H,Dr] and
    band = (origin, pre, next) as in band_mask; ckv_scale None for a bf16 / fp16 latent. Query i of
    sequence b (i < seq_q[b]) attends to latent tokens j < seq_kv[b] that the band leaves visible.
    Returns (out [B,Sq,H,Dn] fp32, lse [B,H,Sq]); with one query token it is mla_decode_attention.
    """
    qn = np.asarray(q_nope, F32)
    qr = np.asarray(q_rope, F32)
    b_cnt, sq, h, dn = qn.shape
    bs = ckv.shape[1]
    out = np.zeros((b_cnt, sq, h, dn), F32)
    lse = np.full((b_cnt, h, sq), -np.inf, F32)
    for b in range(b_cnt):
        L, lq = int(seq_kv[b]), int(seq_q[b])
        if L <= 0 or lq <= 0:
            continue
        pages = np.asarray(block_table[b][: (L + bs - 1) // bs], np.int64)
        c = np.asarray(ckv[pages], F32).reshape(-1, dn)[:L]
        if ckv_scale is not None:
            c = (c * np.asarray(ckv_scale[pages], F32).reshape(-1)[:L, None]).astype(F32)
        kr = np.asarray(krope[pages], F32).reshape(-1, krope.shape[-1])[:L]
        kk = np.concatenate([c, kr], axis=1)
        vis = band_mask(lq, L, *band)
        for hh in range(h):
            qk = np.concatenate([qn[b, :lq, hh], qr[b, :lq, hh]], axis=1)
            o, l = _softmax_attend(qk, kk, c, scale, vis, sink=None if sink is None else float(sink[hh]))
            out[b, :lq, hh] = o
            lse[b, hh, :lq] = l
    return out, lse


# ----------------------------------------------------------------------------- RMS norm family
def _rms(x: np.ndarray, eps: float) -> np.ndarray:
    """rstd per row of fp32 x: 1 / sqrt(mean(x^2) + eps); the sum in float64, rounded once."""
    ms = (np.sum(x.astype(np.float64) ** 2, axis=-1) / x.shape[-1]).astype(F32)
    return (F32(1.0) / np.sqrt((ms + F32(eps)).astype(F32))).astype(F32)


def add_rms_norm(x1, x2, gamma, epsilon: float = 1e-6, dtype: str = "bf16"):
    """npu_add_rms_norm -> (y, rstd, x).

    Follows python/torchair/_ge_concrete_graph/ge_converter/custom/npu_add_rms_norm.py:4-13 and
    the prototype third_party/ascend/include/ops/op_proto/inc/nn_norm.h:50-58 (y and x in the
    input dtype, rstd fp32). x = x1 + x2 in fp32; the norm uses the unrounded fp32 x;
    y = (x * rstd) * gamma rounded to dtype; rstd has shape x.shape[:-1] + [1].
    """
    x = (np.asarray(x1, F32) + np.asarray(x2, F32)).astype(F32)
    g = np.asarray(gamma, F32)
    rstd = _rms(x, epsilon)
    y = round_to(((x * rstd[..., None]).astype(F32) * g).astype(F32), dtype)
    return y, rstd[..., None], round_to(x, dtype)


def add_rms_norm_dynamic_quant(x1, x2, gamma, smooth_scale1=None, smooth_scale2=None, beta=None,
                               epsilon: float = 1e-6, second: bool = False, dtype: str = "bf16"):
    """npu_add_rms_norm_dynamic_quant -> (y1, y2, x, scale1, scale2); y2 / scale2 are None unless
    `second`.

    Follows .../custom/npu_add_rms_norm_dynamic_quant.py:8-21 and the fusion pattern
    python/torchair/patterns/add_rms_norm_dynamic_quant.py:67-80, which replaces
    npu_add_rms_norm + npu_dynamic_quant(y, smooth_scales) by this op: y (+ beta) is rounded
    to the input dtype before it is quantised, so the fused op equals that composition.
    """
    x = (np.asarray(x1, F32) + np.asarray(x2, F32)).astype(F32)
    rstd = _rms(x, epsilon)
    y = ((x * rstd[..., None]).astype(F32) * np.asarray(gamma, F32)).astype(F32)
    if beta is not None:
        y = (y + np.asarray(beta, F32)).astype(F32)
    y = round_to(y, dtype)
    y1, s1 = dynamic_quant(y, smooth_scale1)
    y2 = s2 = None
    if second:
        y2, s2 = dynamic_quant(y, smooth_scale2)
    return y1, y2, round_to(x, dtype), s1, s2


# ----------------------------------------------------------------------------- KV-cache writers
def nz_index(slot: int, block_size: int, row_bytes: int):
    """PA_NZ cache position of a slot's row: (block, offset); 32-byte piece p of the row sits at
    cache[block, p, offset] of the [num_blocks, row_bytes / 32, block_size, 32 B] layout."""
    return slot // block_size, slot % block_size


def scatter_pa_kv_cache(key, value, key_cache, value_cache, slot_mapping, cache_mode: str = "Norm"):
    """npu_scatter_pa_kv_cache: returns updated copies of (key_cache, value_cache).

    Follows .../custom/npu_scatter_pa_kv_cache.py:44-74 (ge.ScatterPaKvCache, prototype
    experiment_ops.h:3963-4002). Token t's row (all heads) goes to slot slot_mapping[t]; negative
    slots are skipped. 'Norm': cache [blocks, block_size, ...] with the slot's row contiguous;
    'PA_NZ': cache [blocks, row / last, block_size, last] (last = 32 bytes of elements), the
    layout of the reference's smoke test tests/smoke/ge_test.py:253-287.
    """
    out = []
    for src, cache in ((key, key_cache), (value, value_cache)):
        c = np.array(cache, copy=True)
        s = np.asarray(src)
        t = s.shape[0]
        rows = s.reshape(t, -1)
        if cache_mode == "Norm":
            flat = c.reshape(-1, rows.shape[1])
            for i in range(t):
                slot = int(slot_mapping[i])
                if slot >= 0:
                    flat[slot] = rows[i]
        else:
            nb, pieces, bs, last = c.shape
            for i in range(t):
                slot = int(slot_mapping[i])
                if slot >= 0:
                    blk, off = nz_index(slot, bs, 0)
                    c[blk, :, off, :] = rows[i].reshape(pieces, last)
        out.append(c)
    return out[0], out[1]


def interleave_rope(x, cos, sin):
    """RoPE of interleaved pairs: xd = (x[..., 0::2], x[..., 1::2]) concatenated, then
    xd * cos + rotate_half(xd) * sin with rotate_half(u) = (-u[h:], u[:h]) (fp32)."""
    x = np.asarray(x, F32)
    xd = np.concatenate([x[..., 0::2], x[..., 1::2]], axis=-1)
    h = xd.shape[-1] // 2
    rh = np.concatenate([-xd[..., h:], xd[..., :h]], axis=-1)
    return ((xd * np.asarray(cos, F32)).astype(F32) + (rh * np.asarray(sin, F32)).astype(F32)).astype(F32)


def kv_rmsnorm_rope_cache(kv, gamma, cos, sin, index, k_cache, ckv_cache, epsilon: float = 1e-5,
                          cache_mode: str = "PA", k_rope_scale=None, k_rope_offset=None, c_kv_scale=None,
                          c_kv_offset=None, c_kv_token_scale=None, dtype: str = "bf16"):
    """npu_kv_rmsnorm_rope_cache (MLA cache update) -> (k_cache, ckv_cache, k_rope, c_kv[, token scales]).

    Follows .../custom/npu_kv_rmsnorm_rope_cache.py:4-66 (ge.KvRmsNormRopeCache, prototype
    experiment_ops.h:3677-3697) and the meta rule
    python/torchair/_contrib/custom_torch_ops/auto_register_custom_torch_ops.py:82-110:
    kv [B, 1, S, dc + dr] splits into the latent (RMS norm with gamma, eps) and the rope key
    (interleaved RoPE with cos / sin [B, 1, S, dr]); both are rounded to the kv dtype and written
    at the token's cache row: PA layouts (cache [blocks, block_size, 1, d]) take index as the
    slot; 'Norm' (cache [B, 1, S_cache, d]) as the position in the token's batch. Negative
    index skips the write. int8 caches: static per-channel round(v * scale + offset) clamped to
    [-128, 127]; for the latent, c_kv_token_scale ([blocks, block_size] fp32) selects per-token
    dynamic quantisation (npu_dynamic_quant arithmetic), its scale stored at the row.
    """
    kv = np.asarray(kv, F32)
    b, n, s, w = kv.shape
    dr = np.asarray(cos).shape[-1]
    dc = w - dr
    flat = kv.reshape(b * s, w)
    lat = flat[:, :dc]
    rstd = _rms(lat, epsilon)
    c_kv = round_to(((lat * rstd[:, None]).astype(F32) * np.asarray(gamma, F32)).astype(F32), dtype)
    k_rope = round_to(interleave_rope(flat[:, dc:], np.asarray(cos, F32).reshape(b * s, dr),
                                      np.asarray(sin, F32).reshape(b * s, dr)), dtype)
    kc = np.array(k_cache, copy=True)
    cc = np.array(ckv_cache, copy=True)
    ts = None if c_kv_token_scale is None else np.array(c_kv_token_scale, F32, copy=True).reshape(-1)
    kflat = kc.reshape(-1, dr)
    cflat = cc.reshape(-1, dc)
    idx = np.asarray(index, np.int64).reshape(-1)
    norm_rows = kc.shape[2] if cache_mode == "Norm" else 0

    def q_static(v, scale, offset):
        o = np.zeros_like(v) if offset is None else np.asarray(offset, F32)
        return np.clip(np.rint((v * np.asarray(scale, F32)).astype(F32) + o), -128, 127).astype(np.int8)

    for t in range(b * s):
        if idx[t] < 0:
            continue
        row = (t // s) * norm_rows + idx[t] if norm_rows else idx[t]
        if kflat.dtype == np.int8:
            kflat[row] = q_static(k_rope[t], k_rope_scale, k_rope_offset)
        else:
            kflat[row] = k_rope[t]
        if cflat.dtype == np.int8:
            if ts is not None:
                q, sc = _quant_rows(c_kv[t][None, :])
                cflat[row] = q[0]
                ts[row] = sc[0]
            else:
                cflat[row] = q_static(c_kv[t], c_kv_scale, c_kv_offset)
        else:
            cflat[row] = c_kv[t]
    out = (kc, cc, k_rope.reshape(b, n, s, dr), c_kv.reshape(b, n, s, dc))
    if ts is not None:
        out = out + (ts.reshape(np.asarray(c_kv_token_scale).shape),)
    return out


# ----------------------------------------------------------------------------- fused MoE grouped GEMMs
def grouped_matmul_swiglu_quant(x, w, weight_scale, x_scale, group_list, group_list_type: int = 0):
    """npu_grouped_matmul_swiglu_quant_v2 (dequant_mode 0, per-token int8) -> (y int8 [m, n/2], scale [m]).

    Follows .../custom/grouped_matmul_swiglu_quant_v2.py:86-166 (ge.GroupedMatmulSwigluQuantV2,
    prototype fusion_ops.h:769-789): the int32 grouped product of npu_grouped_matmul, then
    npu_dequant_swiglu_quant's arithmetic with activate_left (silu of the first half times the second
    half), per-group weight scales and the per-token x_scale; rows past the grouped total give 0.
    """
    x = np.asarray(x)
    m = x.shape[0]
    acc = grouped_matmul(x, w, group_list, group_list_type, out_dtype="int32")
    b, en = group_offsets(group_list, group_list_type, m)
    counts = (en - b).astype(np.int64)
    return dequant_swiglu_quant(acc, np.asarray(weight_scale, F32), np.asarray(x_scale, F32), None, None, counts,
                                activate_left=True)


def grouped_matmul_finalize_routing(x, w, group_list, group_list_type: int = 1, scale=None, pertoken_scale=None,
                                    bias=None, logit=None, row_index=None, shared_input=None,
                                    shared_input_weight: float = 1.0, shared_input_offset: int = 0,
                                    output_bs: int = 0) -> np.ndarray:
    """npu_grouped_matmul_finalize_routing -> y fp32 [output_bs, n].

    Follows .../custom/grouped_matmul_finalize_routing.py:32-133 (ge.GroupedMatmulFinalizeRouting,
    prototype fusion_ops.h:640-725): v[r] = the fp32 dequantised grouped product of row r;
    y[row_index[r]] += logit[r] * v[r], summed over a token's rows in ascending r; shared_input
    rows times shared_input_weight are added at rows [shared_input_offset, + rows).
    """
    x = np.asarray(x)
    m = x.shape[0]
    v = grouped_matmul(x, w, group_list, group_list_type, scale, pertoken_scale, bias, out_dtype="fp32")
    n = v.shape[1]
    bs = output_bs or m
    y = np.zeros((bs, n), F32)
    ri = np.arange(m) if row_index is None else np.asarray(row_index, np.int64)
    lg = np.ones(m, F32) if logit is None else np.asarray(logit, F32)
    for r in range(m):
        t = int(ri[r])
        if 0 <= t < bs:
            y[t] = (y[t] + (lg[r] * v[r]).astype(F32)).astype(F32)
    if shared_input is not None:
        s = np.asarray(shared_input, F32)
        y[shared_input_offset:shared_input_offset + s.shape[0]] = (
            y[shared_input_offset:shared_input_offset + s.shape[0]] + (F32(shared_input_weight) * s).astype(F32))
    return y


def swiglu(x, dim: int = -1, out_dtype: str = "fp32"):
    """npu_swiglu (converter .../custom/npu_swiglu.py:4-14, ge.SwiGlu): y = silu(a) * b, where a and b
    are the first and second halves of x along `dim`, in fp32, rounded once to the output dtype
    ("bf16" / "fp16" / "fp32"). Which half is activated is the operator's documented convention (the
    reference holds only the converter); pinned by reductions in the tests (b = 1 gives silu(a), a = 0
    gives 0, a large gives about a * b)."""
    x = np.asarray(x, F32)
    n = x.shape[dim] // 2
    a = np.take(x, np.arange(n), axis=dim)
    b = np.take(x, np.arange(n, 2 * n), axis=dim)
    with np.errstate(over="ignore"):
        y = ((a / (F32(1) + np.exp(-a))) * b).astype(F32)
    return round_to(y, out_dtype)


def moe_compute_expert_tokens(sorted_experts, num_experts: int):
    """npu_moe_compute_expert_tokens (converter .../custom/npu_moe_compute_expert_tokens.py:4-11,
    prototype experiment_ops.h:3550-3563: "finds the position of the last row processed by each expert
    in the sorted_experts array"): out[e] = the number of entries of the ascending array that are <= e,
    int32 [num_experts]."""
    se = np.asarray(sorted_experts, np.int64)
    return np.searchsorted(se, np.arange(num_experts, dtype=np.int64), side="right").astype(np.int32)

