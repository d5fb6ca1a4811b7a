"""torch.library ops of the RMS-norm family and the KV-cache writers (libtai_kernels.so).

Schemas follow the ops TorchAir's converters accept:
  npu_add_rms_norm                 .../ge_converter/custom/npu_add_rms_norm.py:4-13
  npu_add_rms_norm_dynamic_quant   .../ge_converter/custom/npu_add_rms_norm_dynamic_quant.py:8-21
  npu_scatter_pa_kv_cache(_functional)  .../ge_converter/custom/npu_scatter_pa_kv_cache.py:44-74
  npu_kv_rmsnorm_rope_cache(_v2, _v2_functional)
                                   .../ge_converter/custom/npu_kv_rmsnorm_rope_cache.py:4-66,
                                   python/torchair/_acl_concrete_graph/graph_pass.py:160-163,
                                   python/torchair/_contrib/custom_torch_ops/auto_register_custom_torch_ops.py:16-19, 82-110
In-place variants mutate the caches they are given; functional variants clone them first.
"""
from __future__ import annotations

import math
from typing import List, Optional

import torch

from . import _lib
from ._lib import DT_INT8, DT_NONE
from ._ops_impl import _DT, _check, _define, _f32, _on_gpu, _p, _stream

CACHE_NORM, CACHE_PA_NZ = 0, 1


# ============================================================================ npu_add_rms_norm
def _rstd_shape(x1, gamma):
    nd = max(gamma.dim(), 1)
    return list(x1.shape[:x1.dim() - nd]) + [1] * nd


def _add_rms_norm_fake(x1, x2, gamma, epsilon=1e-6):
    return (torch.empty_like(x1), torch.empty(_rstd_shape(x1, gamma), dtype=torch.float32, device=x1.device),
            torch.empty_like(x1))


def _norm_inputs(name, x1, x2, gamma):
    _on_gpu(x1, x2, gamma)
    _check(x1.dtype in (torch.bfloat16, torch.float16, torch.float32), f"{name}: x1 must be bf16, fp16 or fp32")
    _check(x2.dtype == x1.dtype and gamma.dtype == x1.dtype, f"{name}: x1, x2 and gamma must share a dtype")
    _check(x1.shape == x2.shape, f"{name}: x1 and x2 must have the same shape")
    _check(gamma.dim() >= 1 and tuple(x1.shape[x1.dim() - gamma.dim():]) == tuple(gamma.shape),
           f"{name}: gamma must match the trailing dims of x1")
    cols = gamma.numel()
    rows = x1.numel() // cols if cols else 0
    return x1.contiguous(), x2.contiguous(), gamma.contiguous(), rows, cols


def _add_rms_norm_cuda(x1, x2, gamma, epsilon=1e-6):
    """npu_add_rms_norm -> (y, rstd, x) (npu_add_rms_norm.py:4-13; prototype nn_norm.h:50-58)."""
    a, b, g, rows, cols = _norm_inputs("npu_add_rms_norm", x1, x2, gamma)
    y, rstd, x = _add_rms_norm_fake(a, b, g)
    if rows:
        _lib.call("tai_add_rms_norm", _p(a), _p(b), _p(g), _DT[a.dtype], rows, cols, float(epsilon), _p(y),
                  _p(rstd), _p(x), _stream(a))
    return y, rstd, x


_define("npu", "npu_add_rms_norm(Tensor x1, Tensor x2, Tensor gamma, float epsilon=1e-06) -> (Tensor, Tensor, Tensor)",
        _add_rms_norm_fake, _add_rms_norm_cuda)


# ============================================================================ npu_add_rms_norm_dynamic_quant
def _arnq_fake(x1, x2, gamma, *, smooth_scale1=None, smooth_scale2=None, beta=None, epsilon=1e-6, output_mask=()):
    i8 = torch.empty(x1.shape, dtype=torch.int8, device=x1.device)
    sc = torch.empty(x1.shape[:-1], dtype=torch.float32, device=x1.device)
    return i8, torch.empty_like(i8), torch.empty_like(x1), sc, torch.empty_like(sc)


def _arnq_cuda(x1, x2, gamma, *, smooth_scale1=None, smooth_scale2=None, beta=None, epsilon=1e-6, output_mask=()):
    """npu_add_rms_norm_dynamic_quant -> (y1, y2, x, scale1, scale2)
    (npu_add_rms_norm_dynamic_quant.py:8-21). The second quantisation runs when output_mask[1]
    is set (or, without a mask, when smooth_scale2 is given); otherwise y2 / scale2 are left
    unwritten, as the pattern pass's output_mask=[True, False] asks."""
    name = "npu_add_rms_norm_dynamic_quant"
    a, b, g, rows, cols = _norm_inputs(name, x1, x2, gamma)
    _check(gamma.dim() == 1, f"{name}: gamma must be 1-D (per-row quantisation over the last dim)")
    mask = list(output_mask or [])
    _check(len(mask) in (0, 2), f"{name}: output_mask must have two entries")
    _check(not mask or mask[0], f"{name}: output_mask[0] = False is not supported")
    second = bool(mask[1]) if mask else smooth_scale2 is not None
    bt = None
    if beta is not None:
        _on_gpu(beta)
        _check(beta.dtype == a.dtype and beta.numel() == cols, f"{name}: beta must be [H] of the input dtype")
        bt = beta.contiguous()
    s1, s2 = _f32(smooth_scale1), _f32(smooth_scale2)
    for s in (s1, s2):
        if s is not None:
            _on_gpu(s)
            _check(s.numel() == cols, f"{name}: smooth scales must have H entries")
    y1, y2, x, sc1, sc2 = _arnq_fake(a, b, g)
    if rows:
        _lib.call("tai_add_rms_norm_dynamic_quant", _p(a), _p(b), _p(g), _p(bt), _p(s1), _p(s2) if second else None,
                  _DT[a.dtype], rows, cols, float(epsilon), _p(y1), _p(y2) if second else None, _p(x), _p(sc1),
                  _p(sc2) if second else None, _stream(a))
    return y1, y2, x, sc1, sc2


_define("npu", "npu_add_rms_norm_dynamic_quant(Tensor x1, Tensor x2, Tensor gamma, *, Tensor? smooth_scale1=None, "
               "Tensor? smooth_scale2=None, Tensor? beta=None, float epsilon=1e-06, bool[] output_mask=[]) "
               "-> (Tensor, Tensor, Tensor, Tensor, Tensor)",
        _arnq_fake, _arnq_cuda)


# ============================================================================ npu_scatter_pa_kv_cache
def _cache_geometry(name, src, cache, cache_mode):
    """(num_blocks, block_size, layout code) of a cache for rows shaped like src[t]."""
    row_el = src[0].numel() if src.shape[0] else math.prod(src.shape[1:])
    es = src.element_size()
    _check(cache.dtype == src.dtype, f"{name}: a cache must have its source's dtype")
    _check(cache.is_contiguous(), f"{name}: caches must be contiguous")
    if cache_mode == "PA_NZ":
        last = 32 // es
        _check(cache.dim() == 4 and cache.shape[3] == last and cache.shape[1] * last == row_el,
               f"{name}: PA_NZ cache must be [blocks, row / {last}, block_size, {last}]")
        return cache.shape[0], cache.shape[2], CACHE_PA_NZ
    _check(cache_mode in ("Norm", "PA", "PA_BNSD"), f"{name}: cache_mode {cache_mode!r} not supported "
                                                    "(Norm or PA_NZ)")
    _check(cache.dim() >= 2 and math.prod(cache.shape[2:]) == row_el,
           f"{name}: cache must be [blocks, block_size, ...] with one token row per slot")
    return cache.shape[0], cache.shape[1], CACHE_NORM


def _scatter_into(key, value, key_cache, value_cache, slot_mapping, compress_lens, compress_seq_offsets, seq_lens,
                  cache_mode):
    name = "npu_scatter_pa_kv_cache"
    _on_gpu(key, value, key_cache, value_cache, slot_mapping)
    _check(compress_lens is None and compress_seq_offsets is None and seq_lens is None,
           f"{name}: compress_lens / compress_seq_offsets / seq_lens (compressed caches) are not supported")
    _check(slot_mapping.dtype in (torch.int32, torch.int64), f"{name}: slot_mapping must be int32 or int64")
    _check(key.shape[0] == value.shape[0] == slot_mapping.numel(), f"{name}: one slot per token")
    k, v = key.contiguous(), value.contiguous()
    kb, kbs, kmode = _cache_geometry(name, k, key_cache, cache_mode)
    vb, vbs, _ = _cache_geometry(name, v, value_cache, cache_mode)
    _check(kb == vb and kbs == vbs, f"{name}: key and value caches must have the same blocks")
    t = k.shape[0]
    if t:
        sm = slot_mapping.contiguous()
        _lib.call("tai_scatter_pa_kv_cache", _p(k), _p(v), _p(key_cache), _p(value_cache), _p(sm), _DT[sm.dtype], t,
                  k[0].numel() * k.element_size(), v[0].numel() * v.element_size(), kb, kbs, kmode, _stream(k))


def _scatter_fake(key, value, key_cache, value_cache, slot_mapping, *, compress_lens=None, compress_seq_offsets=None,
                  seq_lens=None, cache_mode="Norm"):
    return None


def _scatter_cuda(key, value, key_cache, value_cache, slot_mapping, *, compress_lens=None, compress_seq_offsets=None,
                  seq_lens=None, cache_mode="Norm"):
    """npu_scatter_pa_kv_cache (in place; ge.ScatterPaKvCache, npu_scatter_pa_kv_cache.py:44-74)."""
    _scatter_into(key, value, key_cache, value_cache, slot_mapping, compress_lens, compress_seq_offsets, seq_lens,
                  cache_mode)


def _scatter_functional_fake(key, value, key_cache, value_cache, slot_mapping, *, compress_lens=None,
                             compress_seq_offsets=None, seq_lens=None, cache_mode="Norm"):
    return torch.empty_like(key_cache), torch.empty_like(value_cache)


def _scatter_functional_cuda(key, value, key_cache, value_cache, slot_mapping, *, compress_lens=None,
                             compress_seq_offsets=None, seq_lens=None, cache_mode="Norm"):
    """npu_scatter_pa_kv_cache_functional: the same writes into copies of the caches."""
    kc, vc = key_cache.clone(), value_cache.clone()
    _scatter_into(key, value, kc, vc, slot_mapping, compress_lens, compress_seq_offsets, seq_lens, cache_mode)
    return kc, vc


_SCATTER_TAIL = ("Tensor slot_mapping, *, Tensor? compress_lens=None, Tensor? compress_seq_offsets=None, "
                 "Tensor? seq_lens=None, str cache_mode='Norm')")
_define("npu", "npu_scatter_pa_kv_cache(Tensor key, Tensor value, Tensor(a!) key_cache, Tensor(b!) value_cache, "
        + _SCATTER_TAIL + " -> ()", _scatter_fake, _scatter_cuda)
_define("npu", "npu_scatter_pa_kv_cache_functional(Tensor key, Tensor value, Tensor key_cache, Tensor value_cache, "
        + _SCATTER_TAIL + " -> (Tensor, Tensor)", _scatter_functional_fake, _scatter_functional_cuda)


# ============================================================================ npu_kv_rmsnorm_rope_cache
def _kv_shapes(kv, gamma, cos, v):
    """(k_rope shape, c_kv shape) of auto_register_custom_torch_ops.py:82-110."""
    if kv.dim() != 4:
        raise RuntimeError("4D tensor expected for input kv")
    if gamma.dim() != 1:
        raise RuntimeError("1D tensor expected for input gamma")
    if cos.dim() != 4:
        raise RuntimeError("4D tensor expected for input cos")
    lead = list(kv.shape[:3])
    if v is None:
        return lead + [cos.shape[3]], lead + [gamma.shape[0]]
    return lead + [kv.shape[3]], lead + [v.shape[3]]


def _kv_write(kv, gamma, cos, sin, index, k_cache, ckv_cache, k_rope_scale, c_kv_scale, k_rope_offset, c_kv_offset,
              v, epsilon, cache_mode):
    """Runs the cache update in place; returns (k_rope, c_kv)."""
    name = "npu_kv_rmsnorm_rope_cache"
    _on_gpu(kv, gamma, cos, sin, index, k_cache, ckv_cache, k_rope_scale, c_kv_scale, k_rope_offset, c_kv_offset)
    _check(v is None, f"{name}: the separate v input is not supported")
    kr_shape, ckv_shape = _kv_shapes(kv, gamma, cos, v)
    _check(kv.shape[1] == 1, f"{name}: kv must have one head ([B, 1, S, D])")
    _check(kv.dtype in (torch.bfloat16, torch.float16, torch.float32), f"{name}: kv must be bf16, fp16 or fp32")
    _check(gamma.dtype == kv.dtype and cos.dtype == kv.dtype and sin.dtype == kv.dtype,
           f"{name}: gamma, cos and sin must have the kv dtype")
    b, _, s, w = kv.shape
    dr = cos.shape[3]
    dc = w - dr
    _check(dc == gamma.shape[0], f"{name}: kv's last dim must be gamma's size plus the rope size")
    _check(tuple(cos.shape) == (b, 1, s, dr) and cos.shape == sin.shape, f"{name}: cos / sin must be [B, 1, S, Dr]")
    _check(index.dtype == torch.int64 and index.numel() == b * s, f"{name}: index must be int64 with B*S entries")
    _check(k_cache.is_contiguous() and ckv_cache.is_contiguous(), f"{name}: caches must be contiguous")
    _check(k_cache.numel() % dr == 0 and ckv_cache.numel() % dc == 0, f"{name}: cache rows must be Dr / Dc wide")
    rows_k, rows_c = k_cache.numel() // dr, ckv_cache.numel() // dc
    _check(rows_k == rows_c, f"{name}: k_cache and ckv_cache must hold the same rows")
    if cache_mode == "Norm":
        _check(k_cache.dim() == 4 and k_cache.shape[0] == b and k_cache.shape[1] == 1,
               f"{name}: Norm caches must be [B, 1, S_cache, D]")
        norm_rows = k_cache.shape[2]
    else:
        _check(cache_mode in ("PA", "PA_BNSD", "PA_BLK_BNSD"),
               f"{name}: cache_mode {cache_mode!r} not supported (Norm, PA, PA_BNSD, PA_BLK_BNSD)")
        norm_rows = 0
    _check(k_cache.dtype in (kv.dtype, torch.int8) and ckv_cache.dtype in (kv.dtype, torch.int8),
           f"{name}: caches must have the kv dtype or int8")
    ks, ko = _f32(k_rope_scale), _f32(k_rope_offset)
    if k_cache.dtype == torch.int8:
        _check(ks is not None and ks.numel() == dr, f"{name}: an int8 k_cache needs k_rope_scale [Dr]")
        _check(ko is None or ko.numel() == dr, f"{name}: k_rope_offset must be [Dr]")
    cs = co = tok = None
    if ckv_cache.dtype == torch.int8:
        _check(c_kv_scale is not None, f"{name}: an int8 ckv_cache needs c_kv_scale")
        if c_kv_scale.numel() == rows_c and (c_kv_scale.dim() >= 2 or rows_c != dc):
            # per-token scale cache ([blocks, block_size] fp32): dynamic quantisation, scale stored
            _check(c_kv_scale.dtype == torch.float32 and c_kv_scale.is_contiguous(),
                   f"{name}: a per-token c_kv_scale cache must be contiguous fp32")
            _check(c_kv_offset is None, f"{name}: per-token quantisation is symmetric (no c_kv_offset)")
            tok = c_kv_scale
        else:
            cs, co = _f32(c_kv_scale), _f32(c_kv_offset)
            _check(cs.numel() == dc and (co is None or co.numel() == dc), f"{name}: c_kv_scale / offset must be [Dc]")
    k_rope = torch.empty(kr_shape, dtype=kv.dtype, device=kv.device)
    c_kv = torch.empty(ckv_shape, dtype=kv.dtype, device=kv.device)
    if b * s:
        kvc, g, cc, sc, ix = kv.contiguous(), gamma.contiguous(), cos.contiguous(), sin.contiguous(), index.contiguous()
        _lib.call("tai_kv_rmsnorm_rope_cache", _p(kvc), _p(g), _p(cc), _p(sc), _p(ix), _DT[kv.dtype], b * s, s, dc, dr,
                  float(epsilon), _p(k_cache), _DT[k_cache.dtype], _p(ckv_cache), _DT[ckv_cache.dtype], rows_c, norm_rows,
                  _p(ks), _p(ko), _p(cs), _p(co), _p(tok), _p(k_rope), _p(c_kv), _stream(kv))
    return k_rope, c_kv


_KV_HEAD = "npu_kv_rmsnorm_rope_cache{sfx}(Tensor kv, Tensor gamma, Tensor cos, Tensor sin, Tensor index, "
_KV_TAIL = ("Tensor? k_rope_offset=None, Tensor? c_kv_offset=None, Tensor? v=None, float epsilon=1e-05, "
            "str cache_mode='Norm', bool is_output_kv=False)")


def _kv_v2_fake(kv, gamma, cos, sin, index, k_cache, ckv_cache, *, k_rope_scale=None, c_kv_scale=None,
                k_rope_offset=None, c_kv_offset=None, v=None, epsilon=1e-5, cache_mode="Norm", is_output_kv=False):
    kr, ckv = _kv_shapes(kv, gamma, cos, v)
    return (torch.empty(kr, dtype=kv.dtype, device=kv.device), torch.empty(ckv, dtype=kv.dtype, device=kv.device))


def _kv_v2_cuda(kv, gamma, cos, sin, index, k_cache, ckv_cache, *, k_rope_scale=None, c_kv_scale=None,
                k_rope_offset=None, c_kv_offset=None, v=None, epsilon=1e-5, cache_mode="Norm", is_output_kv=False):
    """npu_kv_rmsnorm_rope_cache_v2: updates k_cache / ckv_cache (and a per-token c_kv_scale
    cache) in place; returns (k_rope, c_kv)."""
    return _kv_write(kv, gamma, cos, sin, index, k_cache, ckv_cache, k_rope_scale, c_kv_scale, k_rope_offset,
                     c_kv_offset, v, epsilon, cache_mode)


def _kv_v2f_fake(kv, gamma, cos, sin, index, k_cache, ckv_cache, *, k_rope_scale=None, c_kv_scale=None,
                 k_rope_offset=None, c_kv_offset=None, v=None, epsilon=1e-5, cache_mode="Norm", is_output_kv=False):
    kr, ckv = _kv_v2_fake(kv, gamma, cos, sin, index, k_cache, ckv_cache, v=v)
    return kr, ckv, torch.empty_like(k_cache), torch.empty_like(ckv_cache)


def _functional_scale(name, c_kv_scale, ckv_cache):
    _check(not (ckv_cache.dtype == torch.int8 and c_kv_scale is not None and c_kv_scale.dim() >= 2),
           f"{name}: the functional form cannot update a per-token scale cache; use the in-place op")


def _kv_v2f_cuda(kv, gamma, cos, sin, index, k_cache, ckv_cache, *, k_rope_scale=None, c_kv_scale=None,
                 k_rope_offset=None, c_kv_offset=None, v=None, epsilon=1e-5, cache_mode="Norm", is_output_kv=False):
    """npu_kv_rmsnorm_rope_cache_v2_functional -> (k_rope, c_kv, k_cache', ckv_cache')
    (the output order of npu_kv_rmsnorm_rope_cache.py:31-66)."""
    _functional_scale("npu_kv_rmsnorm_rope_cache_v2_functional", c_kv_scale, ckv_cache)
    kc, cc = k_cache.clone(), ckv_cache.clone()
    kr, ckv = _kv_write(kv, gamma, cos, sin, index, kc, cc, k_rope_scale, c_kv_scale, k_rope_offset, c_kv_offset, v,
                        epsilon, cache_mode)
    return kr, ckv, kc, cc


def _kv_legacy_fake(kv, gamma, cos, sin, index, k_cache, ckv_cache, *, k_rope_scale=None, c_kv_scale=None,
                    k_rope_offset=None, c_kv_offset=None, v=None, epsilon=1e-5, cache_mode="Norm", is_output_kv=False):
    kr, ckv = _kv_v2_fake(kv, gamma, cos, sin, index, k_cache, ckv_cache, v=v)
    return torch.empty_like(k_cache), torch.empty_like(ckv_cache), kr, ckv


def _kv_legacy_cuda(kv, gamma, cos, sin, index, k_cache, ckv_cache, *, k_rope_scale=None, c_kv_scale=None,
                    k_rope_offset=None, c_kv_offset=None, v=None, epsilon=1e-5, cache_mode="Norm", is_output_kv=False):
    """npu_kv_rmsnorm_rope_cache -> (k_cache', ckv_cache', k_rope, c_kv), the meta rule of
    auto_register_custom_torch_ops.py:82-110 (new cache tensors)."""
    _functional_scale("npu_kv_rmsnorm_rope_cache", c_kv_scale, ckv_cache)
    kc, cc = k_cache.clone(), ckv_cache.clone()
    kr, ckv = _kv_write(kv, gamma, cos, sin, index, kc, cc, k_rope_scale, c_kv_scale, k_rope_offset, c_kv_offset, v,
                        epsilon, cache_mode)
    return kc, cc, kr, ckv


_define("npu", _KV_HEAD.format(sfx="_v2") + "Tensor(a!) k_cache, Tensor(b!) ckv_cache, *, Tensor? k_rope_scale=None, "
        "Tensor(c!)? c_kv_scale=None, " + _KV_TAIL + " -> (Tensor, Tensor)", _kv_v2_fake, _kv_v2_cuda)
_define("npu", _KV_HEAD.format(sfx="_v2_functional") + "Tensor k_cache, Tensor ckv_cache, *, "
        "Tensor? k_rope_scale=None, Tensor? c_kv_scale=None, " + _KV_TAIL + " -> (Tensor, Tensor, Tensor, Tensor)",
        _kv_v2f_fake, _kv_v2f_cuda)
_LEGACY = (_KV_HEAD.format(sfx="") + "Tensor k_cache, Tensor ckv_cache, *, Tensor? k_rope_scale=None, "
           "Tensor? c_kv_scale=None, " + _KV_TAIL + " -> (Tensor, Tensor, Tensor, Tensor)")
_define("npu", _LEGACY, _kv_legacy_fake, _kv_legacy_cuda)
_define("npu_inference", _LEGACY, _kv_legacy_fake, _kv_legacy_cuda)
