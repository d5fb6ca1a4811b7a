"""npu_fused_infer_attention_score: output-shape rules and dispatch onto the HIP kernels.

Output shapes follow python/torchair/ops/_npu_fused_infer_attention_score.py:160-374
(layout table, value head dim, attention_out and softmax_lse shapes). The ROCm
implementation serves four cases:
  * paged GQA decode    - block_table given, one query token per sequence that sees the whole cached
                          prefix;
  * paged query sequences - block_table given, several query tokens (chunked prefill, multi-token
                          decode) or a band mask: the prefill kernel reading K/V through the block table;
  * MLA absorbed decode - block_table + query_rope/key_rope, int8 latent cache with a
                          per-token fp32 scale (key_antiquant_mode 1);
  * dense prefill       - no block_table.
Masks: sparse_mode 2 / 3 (causal from the top-left / bottom-right), 0 and 4 (a band of pre_tokens /
next_tokens from the top-left / bottom-right).
Sequence lengths stay on the device (tensor arguments of air::npu_fused_infer_attention_score),
so a captured graph replays correctly with new lengths.
"""
from __future__ import annotations

import ctypes
import types
from typing import Dict, Optional, Tuple

import torch

from . import _lib
from ._lib import DT_BF16, DT_FP16, DT_NONE

# input_layout -> (query layout, output layout, query rank)
_LAYOUTS: Dict[str, Tuple[str, str, int]] = {
    "BSH": ("BSH", "BSH", 3), "BSND": ("BSND", "BSND", 4), "BNSD": ("BNSD", "BNSD", 4),
    "TND": ("TND", "TND", 3), "NTD": ("NTD", "NTD", 3), "BNSD_BSND": ("BNSD", "BSND", 4),
    "BSH_BNSD": ("BSH", "BNSD", 3), "BSND_BNSD": ("BSND", "BNSD", 4), "NTD_TND": ("NTD", "TND", 3),
    "BSH_NBSD": ("BSH", "NBSD", 3), "BSND_NBSD": ("BSND", "NBSD", 4), "BNSD_NBSD": ("BNSD", "NBSD", 4),
    "TND_NTD": ("TND", "NTD", 3), "NSD": ("NSD", "NSD", 3),
}


def _layouts(query, input_layout):
    if input_layout not in _LAYOUTS:
        raise ValueError(f"Layout {input_layout} is not supported!")
    ql, ol, qdim = _LAYOUTS[input_layout]
    if query.dim() != qdim:
        raise ValueError(f"Layout {ql}, queryDims({query.dim()}) must be {qdim}!")
    return ql, ol


def _bsnd(query, ql, num_heads):
    """(batch, seq, heads, head_dim) of the query in layout ql."""
    if ql == "BSH":
        return query.size(0), query.size(1), num_heads, query.size(2) // num_heads
    if ql == "BSND":
        return query.size(0), query.size(1), query.size(2), query.size(3)
    if ql == "BNSD":
        return query.size(0), query.size(2), query.size(1), query.size(3)
    if ql == "NSD":
        return 1, query.size(1), query.size(0), query.size(2)
    raise ValueError(f"Layout {ql} is not supported in get_query_b_s_n_d function!")


def _tnd(query, ql):
    if ql == "TND":
        return query.size(0), query.size(1), query.size(2)
    if ql == "NTD":
        return query.size(1), query.size(0), query.size(2)
    raise ValueError(f"Layout {ql} is not supported in get_query_t_n_d function!")


def _value_d(block_table, value, query, ql, n_kv):
    if block_table is not None:
        if value.dim() == 3:
            return value.size(2) // n_kv
        if value.dim() == 4:
            return value.size(3)
        if value.dim() == 5:
            return value.size(2) * value.size(4)
        raise ValueError(f"when Page Attention enabled, value dim should be 3/4/5, but got {value.dim()}!")
    if value.dim() != query.dim():
        raise ValueError(f"when Page Attention not enabled, value dim{value.dim()} should equal to query dim{query.dim()}!")
    if ql == "BSH":
        return value.size(2) // n_kv
    if ql in ("BNSD", "BSND"):
        return value.size(3)
    return value.size(2)


def _out_shape(ol, query, ql, num_heads, value_d):
    def od(d1):
        return d1 if (value_d == 0 or d1 == 0) else value_d
    if ol in ("TND", "NTD"):
        t, n1, d1 = _tnd(query, ql)
        return [t, n1, od(d1)] if ol == "TND" else [n1, t, od(d1)]
    b, s1, n1, d1 = _bsnd(query, ql, num_heads)
    if ol == "BSH":
        h = n1 * value_d
        return [b, s1, h if (h != 0 and query.size(2) != 0) else query.size(2)]
    if ol == "BSND":
        return [b, s1, n1, od(d1)]
    if ol == "BNSD":
        return [b, n1, s1, od(d1)]
    if ol == "NBSD":
        return [n1, b, s1, od(d1)]
    if ol == "NSD":
        return [n1, s1, od(d1)]
    raise ValueError(f"output layout {ol} not supported")


def _lse_shape(query, input_layout, ql, num_heads):
    if input_layout in ("TND", "NTD", "TND_NTD", "NTD_TND"):
        t, n1, _ = _tnd(query, ql)
        return [t, n1, 1]
    b, s1, n1, _ = _bsnd(query, ql, num_heads)
    return [b, n1, s1, 1]


def fia_fake(query, key, value, **kw):
    num_heads = kw.get("num_heads", 1)
    if num_heads <= 0:
        raise ValueError(f"numHeads should be greater than 0, but got {num_heads}!")
    n_kv = kw.get("num_key_value_heads", 0) or num_heads
    input_layout = kw.get("input_layout", "BSH")
    ql, ol = _layouts(query, input_layout)
    vd = _value_d(kw.get("block_table"), value, query, ql, n_kv)
    if value is not None and value.dtype == torch.int32:  # int4 packed in int32
        vd *= 8
    shape = _out_shape(ol, query, ql, num_heads, vd)
    if kw.get("quant_scale2") is not None:
        dt = torch.int8
    elif query.dtype == torch.int8:
        qr = kw.get("query_rope")
        dt = qr.dtype if qr is not None else torch.half
    else:
        dt = query.dtype
    out = query.new_empty(shape, dtype=dt)
    if kw.get("softmax_lse_flag", False):
        lse = query.new_empty(_lse_shape(query, input_layout, ql, num_heads), dtype=torch.float32)
    else:
        lse = query.new_empty([0], dtype=torch.float32)
    return out, lse


_UNSUPPORTED = ("query_padding_size", "kv_padding_size", "key_rope_antiquant_scale")
_QQ_SCALES = ("dequant_scale1", "quant_scale1", "dequant_scale2")


def _lens_tensor(v, device) -> Optional[torch.Tensor]:
    if v is None:
        return None
    if isinstance(v, torch.Tensor):
        return v.to(device=device, dtype=torch.int64).contiguous()
    vals = tuple(int(x) for x in v)
    if torch.device(device).type == "cuda":
        from .graph import capture_resources, preparing_capture
        pinned = capture_resources()
        key = ("fia_lens", vals)
        if preparing_capture() and pinned is not None and key not in pinned:
            # The list is a constant of the graph about to be captured (other values capture anew).
            # A blocking host-to-device copy cannot be captured, so the captured graph copies the
            # lengths from a pinned host buffer, owned by that graph, which every replay re-reads.
            # It is allocated here, in the warm-up run before the capture: pinned memory cannot be
            # allocated while a stream is captured.
            pinned[key] = torch.tensor(vals, dtype=torch.int64).pin_memory()
        if torch.cuda.is_current_stream_capturing():
            host = pinned.get(key) if pinned is not None else None
            if host is None:
                raise RuntimeError("npu_fused_infer_attention_score: list-valued sequence lengths under hipGraph "
                                   "capture need a warm-up run first (or pass them as a device tensor)")
            out = torch.empty(len(vals), dtype=torch.int64, device=device)
            out.copy_(host, non_blocking=True)
            return out
    return torch.tensor(vals, dtype=torch.int64, device=device)



def _check(cond, msg):
    if not cond:
        raise RuntimeError(msg)


def _strides_bshd(t: torch.Tensor, layout: str, heads: int):
    """Element strides (batch, seq, head) of q/k/v/out in the given layout; the last dim must be dense."""
    _check(t.stride(-1) == 1, "npu_fused_infer_attention_score: head_dim must be contiguous")
    if layout == "BSH":
        d = t.size(2) // heads
        return [t.stride(0), t.stride(1), d]
    if layout == "BSND":
        return [t.stride(0), t.stride(1), t.stride(2)]
    if layout == "BNSD":
        return [t.stride(0), t.stride(2), t.stride(1)]
    if layout == "TND":  # packed rows: no batch stride
        return [0, t.stride(0), t.stride(1)]
    if layout == "NTD":
        return [0, t.stride(1), t.stride(0)]
    raise RuntimeError(f"npu_fused_infer_attention_score: layout {layout} not supported for prefill")


_PACKED = ("TND", "NTD")


def _one_token_each(query, ql, ol, kw, b):
    """A TND query of one token per sequence (T == B and actual_seq_lengths absent or the host list
    1..B), which the one-token kernels serve as [B, N, D]."""
    if ql != "TND" or ol != "TND" or query.size(0) != b:
        return False
    v = kw.get("actual_seq_lengths")
    if v is None:
        return True
    return not isinstance(v, torch.Tensor) and [int(x) for x in v] == list(range(1, b + 1))


def _max_run(cum: torch.Tensor) -> int:
    """The longest sequence of cumulative ends (a host sync; explicit masks are sized against it)."""
    c = [0] + cum.tolist()
    return max([c[i + 1] - c[i] for i in range(len(c) - 1)] + [0])


def fia_cuda(query, key, value, **kw):
    """ROCm implementation of npu_fused_infer_attention_score (fused_infer_attention_score.py:4-109)."""
    for name in _UNSUPPORTED:
        v = kw.get(name)
        _check(v is None or (isinstance(v, (list, tuple)) and len(v) == 0),
               f"npu_fused_infer_attention_score: {name} is not supported")
    for t in (query, key, value):
        _check(t.device.type == "cuda", "npu_fused_infer_attention_score runs on the ROCm device only")
    out, lse = fia_fake(query, key, value, **kw)
    num_heads = kw.get("num_heads", 1)
    n_kv = kw.get("num_key_value_heads", 0) or num_heads
    input_layout = kw.get("input_layout", "BSH")
    ql, ol = _layouts(query, input_layout)
    scale = float(kw.get("scale", 1.0))
    block_table = kw.get("block_table")
    want_lse = bool(kw.get("softmax_lse_flag", False))
    stream = torch.cuda.current_stream(query.device).cuda_stream
    seq_kv = _lens_tensor(kw.get("actual_seq_lengths_kv"), query.device)
    seq_q = _lens_tensor(kw.get("actual_seq_lengths"), query.device)

    mask_origin, pre, nxt, explicit = _mask_params(kw)
    # int8 key / value caches (GQA / MHA) and int8 attention_out take the general kernel
    quant_out = kw.get("quant_scale2") is not None
    kv8 = key.dtype == torch.int8 and kw.get("query_rope") is None
    qq = query.dtype == torch.int8
    _check(qq == all(kw.get(n) is not None for n in _QQ_SCALES) and (qq or all(kw.get(n) is None for n in _QQ_SCALES)),
           "npu_fused_infer_attention_score: an int8 query takes dequant_scale1, quant_scale1 and dequant_scale2 "
           "(and they apply to an int8 query only)")
    if qq:
        _check(kw.get("query_rope") is None and kw.get("pse_shift") is None and kw.get("key_shared_prefix") is None
               and all(kw.get(n) is None for n in ("key_antiquant_scale", "key_antiquant_offset", "value_antiquant_scale",
                                                  "value_antiquant_offset", "antiquant_scale", "antiquant_offset")),
               "npu_fused_infer_attention_score: an int8 query is served for GQA/MHA without antiquant scales, pse_shift "
               "or a shared prefix")
    pse = kw.get("pse_shift")
    _check(pse is None or kw.get("query_rope") is None, "npu_fused_infer_attention_score: pse_shift is served for "
           "GQA/MHA, not MLA")
    prefix = kw.get("key_shared_prefix") is not None
    _check(prefix == (kw.get("value_shared_prefix") is not None), "npu_fused_infer_attention_score: "
           "key_shared_prefix and value_shared_prefix come together")
    _check(not prefix or kw.get("query_rope") is None, "npu_fused_infer_attention_score: a shared prefix is served "
           "for GQA/MHA")
    _check(prefix or kw.get("actual_shared_prefix_len") is None, "npu_fused_infer_attention_score: "
           "actual_shared_prefix_len needs key_shared_prefix")
    sink = kw.get("learnable_sink")  # (the v2 op's input)
    _check(sink is None or not qq, "npu_fused_infer_attention_score: learnable_sink is not served with an int8 query")
    # a sink with nothing else also runs on the one-token decode kernel (its merge takes the sink in);
    # every other case with a prefix or a sink takes the general kernel
    sink_only = pse is None and not prefix and sink is not None
    pse = pse if pse is not None else (True if prefix or sink is not None else None)
    _check(kw.get("quant_offset2") is None or quant_out, "npu_fused_infer_attention_score: quant_offset2 needs "
           "quant_scale2")
    if kw.get("query_rope") is None:
        for name in ("key_antiquant_scale", "key_antiquant_offset", "value_antiquant_scale", "value_antiquant_offset",
                     "antiquant_scale", "antiquant_offset"):
            _check(kw.get(name) is None or kv8, f"npu_fused_infer_attention_score: {name} applies to int8 key/value")
    else:
        for name in ("key_antiquant_offset", "value_antiquant_scale", "value_antiquant_offset", "antiquant_scale",
                     "antiquant_offset"):
            _check(kw.get(name) is None, f"npu_fused_infer_attention_score: {name} is not supported with MLA")
        _check(not quant_out, "npu_fused_infer_attention_score: int8 attention_out (quant_scale2) is served for "
               "GQA/MHA, not MLA")

    if block_table is not None:
        packed = ql in _PACKED and not _one_token_each(query, ql, ol, kw, block_table.size(0))
        _check(packed or (ql in ("BSH", "BSND", "BNSD", "TND") and ol == ql),
               "npu_fused_infer_attention_score: paged attention supports BSH/BSND/BNSD/TND without layout change "
               "(and packed TND/NTD queries)")
        b = block_table.size(0) if packed else query.size(0)
        s = 1 if ql == "TND" else _bsnd(query, ql, num_heads)[1]
        _check(seq_kv is not None and seq_kv.numel() == b,
               "npu_fused_infer_attention_score: actual_seq_lengths_kv is required with block_table")
        bt = block_table.to(torch.int32).contiguous()
        _check(bt.dim() == 2 and bt.size(0) == b, "npu_fused_infer_attention_score: block_table must be [B, max_blocks]")
        if kw.get("query_rope") is not None:
            whole_prefix = pre >= _NO_BOUND and (nxt >= _NO_BOUND or (mask_origin == 1 and nxt >= 0))
            # (the one-token kernel steps through pages 32 tokens at a time; key is [blocks, bs, (1,) Dn])
            if (key.dtype == torch.int8 and s == 1 and whole_prefix and not explicit and key.size(1) % 32 == 0
                    and not packed and sink is None):
                return _mla(query, key, value, kw, out, lse, want_lse, num_heads, n_kv, bt, seq_kv, scale, stream)
            # several query tokens (MTP / speculative decode), bands and masks: the general kernel
            return _general_mla(query, key, value, kw, out, lse, want_lse, ql, num_heads, n_kv, bt, seq_q, seq_kv,
                                scale, mask_origin, pre, nxt, explicit, stream, ol=ol)
        dt = _half_code(query, key, value, kv8)
        d = _value_d(block_table, value, query, ql, n_kv)
        if key.dim() == 3:
            bs = key.size(1)
            _check(key.size(2) == n_kv * d, "npu_fused_infer_attention_score: key cache must be [blocks, bs, Hkv*D]")
            sb, ss, sh = key.stride(0), key.stride(1), d
        else:
            _check(key.dim() == 4 and key.size(1) == n_kv and key.size(3) == d,
                   "npu_fused_infer_attention_score: key cache must be [blocks, Hkv, bs, D]")
            bs = key.size(2)
            sb, ss, sh = key.stride(0), key.stride(2), key.stride(1)
        _check(key.stride(-1) == 1 and value.stride() == key.stride() and value.shape == key.shape,
               "npu_fused_infer_attention_score: key/value caches must share shape and a dense head dim")
        blk = kw.get("block_size", 0) or bs
        _check(blk == bs, "npu_fused_infer_attention_score: block_size does not match the cache")
        whole = s == 1 and pre >= _NO_BOUND and (nxt >= _NO_BOUND or (mask_origin == 1 and nxt >= 0))
        if (kv8 and whole and not explicit and not quant_out and pse is None and bs % 32 == 0 and d in (64, 128, 256)
                and not packed and key.stride(-1) == 1 and value.stride() == key.stride()):
            # one query token over int8 caches with per-channel scales and no offsets: the decode kernel
            aq, keep = types.SimpleNamespace(), []
            _antiquant_params(aq, kw, b, n_kv, d, d, keep)
            if aq.k_quant_mode == 0 and aq.v_quant_mode == 0 and aq.k_offset is None and aq.v_offset is None:
                q = query.contiguous()
                ws_bytes = _lib.query("tai_fia_paged_decode_kv8_workspace_size", b, num_heads, n_kv, d, bt.size(1), bs)
                ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
                _lib.call("tai_fia_paged_decode_kv8", q.data_ptr(), key.data_ptr(), value.data_ptr(), sb, ss, sh,
                          bt.data_ptr(), bt.size(1), seq_kv.data_ptr(), b, num_heads, n_kv, d, dt, bs, scale,
                          aq.k_scale, aq.v_scale, out.data_ptr(), lse.data_ptr() if want_lse else None, ws.data_ptr(),
                          ws_bytes, stream)
                return out, lse
        # the tiled kernels step through pages 32 tokens at a time
        if (explicit or kv8 or quant_out or (pse is not None and not (sink_only and whole)) or bs % 32 != 0
                or d not in (64, 128, 256) or (s > 1 and d not in (64, 128)) or packed):
            kstr = [sb, ss, sh]
            return _general_call(query, key, value, out, lse, want_lse, ql, num_heads, n_kv, d, dt, kstr, kstr,
                                 bt, bs, seq_q, seq_kv, mask_origin, pre, nxt, explicit, kw, scale, stream,
                                 kv8=kv8, quant_out=quant_out, ol=ol)
        # one query token that the mask leaves the whole prefix: the decode kernel
        if whole:
            q = query.contiguous()
            ws_bytes = _lib.query("tai_fia_paged_decode_workspace_size", b, num_heads, d, bt.size(1), bs)
            ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
            head = (q.data_ptr(), key.data_ptr(), value.data_ptr(), sb, ss, sh, bt.data_ptr(), bt.size(1),
                    seq_kv.data_ptr(), b, num_heads, n_kv, d, dt, bs, scale)
            tail = (out.data_ptr(), lse.data_ptr() if want_lse else None, ws.data_ptr(), ws_bytes, stream)
            if sink is not None:
                sk = sink.to(torch.float32).reshape(-1).contiguous()
                _check(sk.numel() == num_heads, f"npu_fused_infer_attention_score: learnable_sink must hold one logit "
                       f"per query head ({num_heads}), got {sk.numel()}")
                _lib.call("tai_fia_paged_decode_sink", *head, sk.data_ptr(), *tail)
            else:
                _lib.call("tai_fia_paged_decode", *head, *tail)
            return out, lse
        # query sequences over the paged cache (chunked prefill, multi-token decode)
        b, s_q, hq, d = _bsnd(query, ql, num_heads)
        qs = _strides_bshd(query, ql, hq)
        os_ = _strides_bshd(out, ol, hq)
        kstr = [0, ss, sh]
        return _prefill_call(query, key, value, out, lse, want_lse, b, s_q, bt.size(1) * bs, hq, n_kv, d, dt, qs, kstr,
                             kstr, os_, seq_q, seq_kv, mask_origin, pre, nxt, bt, bs, sb, sb, scale, stream)

    # ---------------------------------------------------------------- dense prefill
    _check(ql in _PACKED or (ql in ("BSH", "BSND", "BNSD") and ol == ql),
           "npu_fused_infer_attention_score: prefill supports BSH/BSND/BNSD without layout change, and packed "
           "TND/NTD queries")
    _check(kw.get("query_rope") is None, "npu_fused_infer_attention_score: MLA needs a paged latent cache (block_table)")
    dt = _half_code(query, key, value, kv8)
    _dense_kv_check(query, key, value, ql, num_heads, n_kv)
    if ql in _PACKED:
        d = _tnd(query, ql)[2]
        return _general_call(query, key, value, out, lse, want_lse, ql, num_heads, n_kv, d, dt,
                             _strides_bshd(key, ql, n_kv), _strides_bshd(value, ql, n_kv), None, 0, seq_q, seq_kv,
                             mask_origin, pre, nxt, explicit, kw, scale, stream, kv8=kv8, quant_out=quant_out, ol=ol)
    b, s_q, hq, d = _bsnd(query, ql, num_heads)
    if (explicit or kv8 or quant_out or pse is not None or d not in (64, 128)
            or _value_d(None, value, query, ql, n_kv) != d):
        return _general_call(query, key, value, out, lse, want_lse, ql, num_heads, n_kv, d, dt,
                             _strides_bshd(key, ql, n_kv), _strides_bshd(value, ql, n_kv), None, 0, seq_q, seq_kv,
                             mask_origin, pre, nxt, explicit, kw, scale, stream, kv8=kv8, quant_out=quant_out)
    s_kv = key.size(2) if ql == "BNSD" else key.size(1)
    qs = _strides_bshd(query, ql, hq)
    ks = _strides_bshd(key, ql, n_kv)
    vs = _strides_bshd(value, ql, n_kv)
    os_ = _strides_bshd(out, ol, hq)
    return _prefill_call(query, key, value, out, lse, want_lse, b, s_q, s_kv, hq, n_kv, d, dt, qs, ks, vs, os_, seq_q,
                         seq_kv, mask_origin, pre, nxt, None, 0, 0, 0, scale, stream)


# pre_tokens / next_tokens at or above this are no bound (the default 2147483647)
_NO_BOUND = 2147483647


def _mask_params(kw):
    """(origin, pre_tokens, next_tokens) of the attention mask: query i of len_q sees kv j of len_kv when
    -pre <= j - i - off <= next, off = len_kv - len_q (origin 1, bottom-right) or 0 (origin 0, top-left).
    sparse_mode 0: band of pre/next tokens from the top-left (no bound by default); 2: top-left causal;
    3: bottom-right causal; 4: band of pre/next tokens from the bottom-right. Modes 2-4 take the fixed
    compressed triangle as atten_mask (torch_npu's 2048 x 2048 convention); its contents are implied by
    the mode and not read. Modes 0 and 1 read an explicit atten_mask (nonzero = masked out; mode 0 also
    applies the band), which the general kernel serves. Returns (origin, pre, next, explicit)."""
    sparse_mode = int(kw.get("sparse_mode", 0))
    pre = int(kw.get("pre_tokens", _NO_BOUND))
    nxt = int(kw.get("next_tokens", _NO_BOUND))
    explicit = kw.get("atten_mask") is not None and sparse_mode in (0, 1)
    if sparse_mode == 0:
        return 0, pre, nxt, explicit
    if sparse_mode == 1:
        _check(explicit, "npu_fused_infer_attention_score: sparse_mode 1 needs atten_mask")
        return 0, _NO_BOUND, _NO_BOUND, True
    if sparse_mode == 2:
        return 0, _NO_BOUND, 0, False
    if sparse_mode == 3:
        return 1, _NO_BOUND, 0, False
    if sparse_mode == 4:
        return 1, pre, nxt, False
    raise RuntimeError(f"npu_fused_infer_attention_score: sparse_mode {sparse_mode} is not supported (0-4)")


def _mask_bytes(mask, b, s_q):
    """An explicit atten_mask as bytes (nonzero = masked out) with (batch, query, kv) strides; a leading
    batch dim of 1, or none, broadcasts. Shapes [Sq, Skv], [B, Sq, Skv], [B, 1, Sq, Skv]."""
    m = mask if mask.dtype in (torch.bool, torch.uint8, torch.int8) else (mask != 0)
    m = m.to(torch.uint8) if m.dtype == torch.bool else m.view(torch.uint8) if m.dtype == torch.int8 else m
    if m.dim() == 4:
        _check(m.size(1) == 1, "npu_fused_infer_attention_score: atten_mask [B, N, Sq, Skv] needs N == 1")
        m = m[:, 0]
    if m.dim() == 2:
        m = m.unsqueeze(0)
    _check(m.dim() == 3 and m.size(0) in (1, b) and m.size(1) >= s_q,
           "npu_fused_infer_attention_score: atten_mask must be [Sq, Skv], [B, Sq, Skv] or [B, 1, Sq, Skv]")
    m = m.contiguous()
    st = [0 if m.size(0) == 1 else m.stride(0), m.stride(1), m.stride(2)]
    return m, st


def _general_args(dt, b, s_q, s_kv, hq, n_kv, dk1, dk2, dv, q1, q1s, q2, q2s, k1, k1s, k2, k2s, v, vs, bt, bs,
                  seq_q, seq_kv, mask, mask_st, mask_origin, pre, nxt, scale, out, os_, lse):
    a = _lib.FiaGeneralArgs()
    a.dtype, a.dk1, a.dk2, a.dv = dt, dk1, dk2, dv
    a.b, a.s_q, a.s_kv, a.hq, a.hkv = b, s_q, s_kv, hq, n_kv
    a.q1, a.q1_strides = q1.data_ptr(), _lib._I64x3(*q1s)
    a.q2, a.q2_strides = (q2.data_ptr() if q2 is not None else None), _lib._I64x3(*(q2s or [0, 0, 0]))
    a.k1, a.k1_strides = k1.data_ptr(), _lib._I64x3(*k1s)
    a.k2, a.k2_strides = (k2.data_ptr() if k2 is not None else None), _lib._I64x3(*(k2s or [0, 0, 0]))
    a.v, a.v_strides = v.data_ptr(), _lib._I64x3(*vs)
    a.block_table = bt.data_ptr() if bt is not None else None
    a.max_blocks = bt.size(1) if bt is not None else 0
    a.block_size = bs
    a.seq_lens_q = seq_q.data_ptr() if seq_q is not None else None
    a.seq_lens_kv = seq_kv.data_ptr() if seq_kv is not None else None
    a.mask = mask.data_ptr() if mask is not None else None
    a.mask_strides = _lib._I64x3(*(mask_st or [0, 0, 0]))
    a.mask_origin, a.pre_tokens, a.next_tokens, a.scale = mask_origin, pre, nxt, scale
    a.out, a.out_strides = out.data_ptr(), _lib._I64x3(*os_)
    a.lse = lse.data_ptr() if lse is not None else None
    return a


def _antiquant_params(a, kw, b, n_kv, dk, dv, keep):
    """Fills the int8 key/value fields of tai_fia_general_args: (x + offset) * scale per channel (mode 0,
    [Hkv * D] in any layout the op takes: [H], [N, D], [N, 1, D], [1, N, 1, D]) or per token (mode 1,
    [B, S] or [1, B, S]). key_/value_antiquant_* with key_/value_antiquant_mode, or the combined
    antiquant_scale / antiquant_offset of leading dim 2 (key, value) with antiquant_mode
    (experiment_ops.h:3922-3932; the converter passes them on, fused_infer_attention_score.py:16-27)."""
    ks, ko, km = kw.get("key_antiquant_scale"), kw.get("key_antiquant_offset"), int(kw.get("key_antiquant_mode", 0))
    vs, vo, vm = (kw.get("value_antiquant_scale"), kw.get("value_antiquant_offset"),
                  int(kw.get("value_antiquant_mode", 0)))
    if ks is None and vs is None and kw.get("antiquant_scale") is not None:
        both, both_o = kw["antiquant_scale"], kw.get("antiquant_offset")
        _check(both.size(0) == 2 and (both_o is None or both_o.size(0) == 2),
               "npu_fused_infer_attention_score: antiquant_scale / antiquant_offset hold key and value (leading dim 2)")
        ks, vs = both[0], both[1]
        ko, vo = (both_o[0], both_o[1]) if both_o is not None else (None, None)
        km = vm = int(kw.get("antiquant_mode", 0))
    _check(ks is not None and vs is not None, "npu_fused_infer_attention_score: int8 key/value need antiquant scales "
           "(key_antiquant_scale and value_antiquant_scale, or antiquant_scale)")
    _check(km in (0, 1) and vm in (0, 1), "npu_fused_infer_attention_score: antiquant modes 0 (per channel) and 1 "
           "(per token) are supported")
    tok = 0

    def flat(t, mode, d, what):
        nonlocal tok
        if t is None:
            return None
        t = t.to(torch.float32).contiguous()
        if mode == 0:
            _check(t.numel() == n_kv * d, f"npu_fused_infer_attention_score: per-channel {what} needs Hkv * D = "
                   f"{n_kv * d} entries, got {t.numel()}")
            t = t.reshape(-1)
        else:
            _check(t.numel() % b == 0 and t.numel() > 0, f"npu_fused_infer_attention_score: per-token {what} must be "
                   "[B, S] or [1, B, S]")
            t = t.reshape(b, -1)
            _check(tok in (0, t.size(1)), "npu_fused_infer_attention_score: per-token key and value scales must cover "
                   "the same positions")
            tok = t.size(1)
        keep.append(t)
        return t

    a.kv_dtype = _lib.DT_INT8
    for attr, t, mode, d, what in (("k_scale", ks, km, dk, "key scale"), ("k_offset", ko, km, dk, "key offset"),
                                   ("v_scale", vs, vm, dv, "value scale"), ("v_offset", vo, vm, dv, "value offset")):
        f = flat(t, mode, d, what)
        setattr(a, attr, f.data_ptr() if f is not None else None)
    a.k_quant_mode, a.v_quant_mode, a.tok_stride = km, vm, tok


def _prefix_params(a, kw, ql, n_kv, dk, dv, query, keep) -> int:
    """Shared prefix (experiment_ops.h:3933-3935; the converter passes key_shared_prefix,
    value_shared_prefix and actual_shared_prefix_len on, fused_infer_attention_score.py:29-31, 94-109):
    [1, Sp, H] (BSH), [1, Sp, N, D] (BSND) or [1, N, Sp, D] (BNSD) keys and values that precede every
    sequence's own; actual_shared_prefix_len (one value, default Sp) of them are used."""
    kp, vp = kw["key_shared_prefix"], kw["value_shared_prefix"]
    _check(kp.dtype == query.dtype and vp.dtype == query.dtype and kp.size(0) == 1 and vp.size(0) == 1,
           "npu_fused_infer_attention_score: shared prefixes are [1, ...] of the query's dtype")

    def pos_head(t, d):
        if ql == "BSH":
            _check(t.dim() == 3 and t.size(2) == n_kv * d and t.stride(2) == 1,
                   "npu_fused_infer_attention_score: a BSH shared prefix is [1, Sp, Hkv * D]")
            return t.size(1), [t.stride(1), d]
        if ql == "BSND":
            _check(t.dim() == 4 and t.size(2) == n_kv and t.size(3) == d and t.stride(3) == 1,
                   "npu_fused_infer_attention_score: a BSND shared prefix is [1, Sp, Hkv, D]")
            return t.size(1), [t.stride(1), t.stride(2)]
        _check(t.dim() == 4 and t.size(1) == n_kv and t.size(3) == d and t.stride(3) == 1,
               "npu_fused_infer_attention_score: a BNSD shared prefix is [1, Hkv, Sp, D]")
        return t.size(2), [t.stride(2), t.stride(1)]

    sp, ks = pos_head(kp, dk)
    spv, vs = pos_head(vp, dv)
    _check(sp == spv, "npu_fused_infer_attention_score: key and value shared prefixes differ in length")
    ln = kw.get("actual_shared_prefix_len")
    lt = _lens_tensor(ln if ln is not None else [sp], query.device)
    _check(lt.numel() == 1, "npu_fused_infer_attention_score: actual_shared_prefix_len holds one length")
    a.k_prefix, a.v_prefix = kp.data_ptr(), vp.data_ptr()
    a.k_prefix_strides = (ctypes.c_int64 * 2)(*ks)
    a.v_prefix_strides = (ctypes.c_int64 * 2)(*vs)
    a.prefix_len, a.prefix_cap = lt.data_ptr(), sp
    keep.append(lt)
    return sp


def _sink_param(a, kw, hq, keep):
    """learnable_sink (the v2 op's input; prototype experiment_ops.h:3940, bf16): one logit per query
    head that joins the softmax denominator without a value row."""
    t = kw.get("learnable_sink")
    if t is None:
        return
    t = t.to(torch.float32).reshape(-1).contiguous()
    _check(t.numel() == hq, f"npu_fused_infer_attention_score: learnable_sink must hold one logit per query head "
           f"({hq}), got {t.numel()}")
    keep.append(t)
    a.sink = t.data_ptr()


def _one_scale(t, name):
    """One fp32 scale on the device from a float tensor or a UINT64 one carrying an fp32 in its low 32
    bits (the prototype types dequant_scale1 / dequant_scale2 UINT64, experiment_ops.h:3888-3890)."""
    _check(t.numel() == 1, f"npu_fused_infer_attention_score: {name} holds one (per-tensor) value")
    if t.dtype in (torch.int64, torch.uint64):
        t = t.reshape(1).contiguous().view(torch.int32)[0:1].view(torch.float32)
    return t.to(torch.float32).reshape(1).contiguous()


def _out_quant_params(a, kw, hq, dv, keep):
    """int8 attention_out: clamp(rint(o * quant_scale2 + quant_offset2)), per tensor (1 entry) or per
    channel (Hq * Dv entries, channel h * Dv + d) (experiment_ops.h:3943)."""
    qs = kw["quant_scale2"].to(torch.float32).contiguous().reshape(-1)
    _check(qs.numel() in (1, hq * dv), "npu_fused_infer_attention_score: quant_scale2 must have 1 or N * D entries")
    qo = kw.get("quant_offset2")
    if qo is not None:
        qo = qo.to(torch.float32).contiguous().reshape(-1)
        _check(qo.numel() == qs.numel(), "npu_fused_infer_attention_score: quant_offset2 must match quant_scale2")
        keep.append(qo)
    keep.append(qs)
    a.out_dtype, a.out_scale, a.out_scale_len = _lib.DT_INT8, qs.data_ptr(), qs.numel()
    a.out_offset = qo.data_ptr() if qo is not None else None


def _dense_kv_check(query, key, value, ql, num_heads, n_kv):
    """Dense keys and values must hold what the kernels read: the query's batch, num_key_value_heads
    heads, the query's head dim for the key, and the same positions in both."""
    name = "npu_fused_infer_attention_score"
    if ql in _PACKED:
        _, _, dk = _tnd(query, ql)
        _check(key.dim() == 3 and value.dim() == 3, f"{name}: packed keys/values are [T, N, D] ({ql})")
        n_ax, t_ax = (1, 0) if ql == "TND" else (0, 1)
        _check(key.size(n_ax) == n_kv and value.size(n_ax) == n_kv and key.size(2) == dk,
               f"{name}: {ql} keys/values need {n_kv} heads and the key the query's head dim {dk}")
        _check(value.size(t_ax) == key.size(t_ax), f"{name}: keys and values hold different token counts")
        return
    b, _, _, dk = _bsnd(query, ql, num_heads)
    _check(key.dim() == query.dim() and value.dim() == query.dim() and key.size(0) == b and value.size(0) == b,
           f"{name}: keys/values must have the query's layout and batch {b}")
    dv = _value_d(None, value, query, ql, n_kv)
    if ql == "BSH":
        ok = key.size(2) == n_kv * dk and value.size(2) == n_kv * dv and value.size(1) == key.size(1)
    elif ql == "BSND":
        ok = key.shape[2:] == (n_kv, dk) and value.size(2) == n_kv and value.size(1) == key.size(1)
    else:  # BNSD
        ok = key.size(1) == n_kv and key.size(3) == dk and value.size(1) == n_kv and value.size(2) == key.size(2)
    _check(ok, f"{name}: {ql} keys/values need {n_kv} heads of the query's head dim {dk} (key) and matching "
           "positions")


def _one_token_ends(seq_q, bt, t, device):
    """A packed query over a paged cache without actual_seq_lengths holds one token per sequence (T = B,
    the one-token layout): its cumulative ends are 1..B."""
    if seq_q is None and bt is not None and t == bt.size(0):
        return torch.arange(1, t + 1, dtype=torch.int64, device=device)
    return seq_q


def _packed_lens(a, ql, query, bt, seq_q, seq_kv):
    """Packed TND / NTD queries: the sequences' query rows end at the cumulative actual_seq_lengths
    (torch_npu's TND convention); dense keys/values are packed the same way (cumulative
    actual_seq_lengths_kv), a paged cache takes per-sequence actual_seq_lengths_kv. Returns the
    sequence count and the longest query and kv runs (host values, for explicit-mask checks)."""
    _check(seq_q is not None, f"npu_fused_infer_attention_score: {ql} queries need actual_seq_lengths "
           "(cumulative query ends)")
    b = seq_q.numel()
    _check(seq_kv is not None and seq_kv.numel() == b, f"npu_fused_infer_attention_score: {ql} needs "
           "actual_seq_lengths_kv with one entry per sequence")
    if bt is not None:
        _check(bt.size(0) == b, "npu_fused_infer_attention_score: block_table must have a row per sequence")
    a.q_cum, a.seq_lens_q = seq_q.data_ptr(), None
    if bt is None:
        a.kv_cum, a.seq_lens_kv = seq_kv.data_ptr(), None
    return b


def _general_call(query, key, value, out, lse, want_lse, ql, num_heads, n_kv, d, dt, ks, vs, bt, bs, seq_q, seq_kv,
                  mask_origin, pre, nxt, explicit, kw, scale, stream, kv8=False, quant_out=False, ol=None):
    """The general kernel for GQA/MHA: explicit masks, head dims the tiled kernels do not take, int8
    key/value caches, int8 attention_out and packed (TND / NTD) queries."""
    ol = ol or ql
    packed = ql in _PACKED
    if packed:
        _check(kw.get("pse_shift") is None and kw.get("key_shared_prefix") is None,
               f"npu_fused_infer_attention_score: pse_shift and a shared prefix take batched layouts, not {ql}")
        s_q, hq, _ = _tnd(query, ql)
        seq_q = _one_token_ends(seq_q, bt, s_q, query.device)
        b = seq_q.numel() if seq_q is not None else 0
    else:
        b, s_q, hq, _ = _bsnd(query, ql, num_heads)
    dv = _value_d(bt, value, query, ql, n_kv)
    if bt is not None:
        s_kv = bt.size(1) * bs
    elif packed:
        s_kv = key.size(0) if ql == "TND" else key.size(1)
    else:
        s_kv = key.size(2) if ql == "BNSD" else key.size(1)
    a = _general_args(dt, b, s_q, s_kv, hq, n_kv, d, 0, dv, query, _strides_bshd(query, ql, hq), None, None,
                      key, ks, None, None, value, vs, bt, bs, seq_q, seq_kv, None, None, mask_origin, pre, nxt, scale,
                      out, _strides_bshd(out, ol, hq), lse if want_lse else None)
    if packed:
        b = _packed_lens(a, ql, query, bt, seq_q, seq_kv)
    mask = None
    if explicit:
        mask, mst = _mask_bytes(kw["atten_mask"], b, _max_run(seq_q) if packed else s_q)
        a.mask, a.mask_strides = mask.data_ptr(), _lib._I64x3(*mst)
    keep = [mask]  # (and the fp32 copies of the scales) alive until the launch is queued (stream-ordered frees)
    # Masks and position shifts index keys in the concatenated [shared prefix, own keys] space.
    sp = _prefix_params(a, kw, ql, n_kv, d, dv, query, keep) if kw.get("key_shared_prefix") is not None else 0
    if mask is not None:
        kv_max = (_max_run(seq_kv) if packed and bt is None else max(seq_kv.tolist())) if seq_kv is not None else s_kv
        _check(mask.size(2) >= sp + kv_max,
               "npu_fused_infer_attention_score: atten_mask covers fewer kv positions than the sequences hold")
    pse = kw.get("pse_shift")
    if pse is not None:
        _check(pse.dtype == query.dtype and pse.dim() == 4 and pse.size(0) in (1, b) and pse.size(1) == hq
               and pse.size(2) >= s_q and pse.size(3) >= sp + s_kv,
               "npu_fused_infer_attention_score: pse_shift must be [B or 1, N, >= S_q, >= S_kv] of the query's dtype")
        a.pse = pse.data_ptr()
        a.pse_strides = (ctypes.c_int64 * 4)(0 if pse.size(0) == 1 else pse.stride(0), pse.stride(1), pse.stride(2),
                                             pse.stride(3))
    if query.dtype == torch.int8:
        a.kv_dtype, a.q_dtype = _lib.DT_INT8, _lib.DT_INT8
        for attr, name in (("deq_scale1", "dequant_scale1"), ("quant_scale1", "quant_scale1"),
                           ("deq_scale2", "dequant_scale2")):
            t = _one_scale(kw[name], name)
            keep.append(t)
            setattr(a, attr, t.data_ptr())
    elif kv8:
        _check(key.dtype == torch.int8 and value.dtype == torch.int8,
               "npu_fused_infer_attention_score: int8 key needs an int8 value")
        _antiquant_params(a, kw, b, n_kv, d, dv, keep)
    _sink_param(a, kw, hq, keep)
    if quant_out:
        _out_quant_params(a, kw, hq, dv, keep)
    _lib.call("tai_fia_general", ctypes.byref(a), stream)
    return out, lse


def _general_mla(query, key, value, kw, out, lse, want_lse, ql, num_heads, n_kv, bt, seq_q, seq_kv, scale,
                 mask_origin, pre, nxt, explicit, stream, ol=None):
    """MLA on the general kernel: key = [latent | key_rope], value = latent, one kv head. The latent is
    bf16 / fp16, or int8 with one fp32 scale per cache slot (key_antiquant_scale [blocks, bs],
    key_antiquant_mode 1, as for the one-token kernel), then dequantised as latent * scale."""
    q_rope, k_rope = kw["query_rope"], kw.get("key_rope")
    _check(k_rope is not None, "npu_fused_infer_attention_score: MLA needs key_rope")
    _check(n_kv == 1, "npu_fused_infer_attention_score: MLA latent cache has one kv head")
    ol = ol or ql
    packed = ql in _PACKED
    _check(ql in ("BSH", "BSND", "BNSD") or packed, "npu_fused_infer_attention_score: MLA takes BSH/BSND/BNSD or "
           "packed TND/NTD queries")
    kv8 = key.dtype == torch.int8
    dt = _half_code(query, key, value, kv8)
    _check(q_rope.dtype == query.dtype and k_rope.dtype == query.dtype,
           "npu_fused_infer_attention_score: MLA query_rope/key_rope must have the query's dtype")
    if packed:
        s_q, hq, dn = _tnd(query, ql)
        dr = _tnd(q_rope, ql)[2]
        seq_q = _one_token_ends(seq_q, bt, s_q, query.device)
        b = seq_q.numel() if seq_q is not None else 0
    else:
        b, s_q, hq, dn = _bsnd(query, ql, num_heads)
        dr = _bsnd(q_rope, ql, num_heads)[3]
    nblk = key.size(0)
    kc = key.reshape(nblk, -1, dn)
    bs = kc.size(1)
    kr = k_rope.reshape(nblk, bs, dr)
    _check(kc.stride(-1) == 1 and kr.stride(-1) == 1, "npu_fused_infer_attention_score: caches need a dense last dim")
    kst = [kc.stride(0), kc.stride(1), 0]
    a = _general_args(dt, b, s_q, bt.size(1) * bs, hq, 1, dn, dr, dn, query, _strides_bshd(query, ql, hq), q_rope,
                      _strides_bshd(q_rope, ql, hq), kc, kst, kr, [kr.stride(0), kr.stride(1), 0], kc, kst, bt, bs,
                      seq_q, seq_kv, None, None, mask_origin, pre, nxt, scale, out, _strides_bshd(out, ol, hq),
                      lse if want_lse else None)
    if packed:
        b = _packed_lens(a, ql, query, bt, seq_q, seq_kv)
    mask = None
    if explicit:
        mask, mst = _mask_bytes(kw["atten_mask"], b, _max_run(seq_q) if packed else s_q)
        a.mask, a.mask_strides = mask.data_ptr(), _lib._I64x3(*mst)
    ks = None
    if kv8:
        k_scale = kw.get("key_antiquant_scale")
        _check(k_scale is not None and int(kw.get("key_antiquant_mode", 0)) == 1,
               "npu_fused_infer_attention_score: an int8 MLA latent needs per-token key_antiquant_scale "
               "(key_antiquant_mode=1)")
        ks = k_scale.to(torch.float32).contiguous()
        _check(ks.numel() == nblk * bs, "npu_fused_infer_attention_score: key_antiquant_scale must hold one fp32 per "
                                        "cached token ([blocks, bs])")
        a.kv_dtype, a.k_scale, a.v_scale, a.k_quant_mode, a.v_quant_mode = _lib.DT_INT8, ks.data_ptr(), ks.data_ptr(), 2, 2
    keep = []
    _sink_param(a, kw, hq, keep)
    _lib.call("tai_fia_general", ctypes.byref(a), stream)
    return out, lse


def _half_code(query, key, value, kv8=False) -> int:
    """ScalarType code of the attention element type: bf16 or fp16, the same for query, key and value
    (kv8: int8 key and value caches beside a bf16 / fp16 query)."""
    if query.dtype == torch.int8:  # the meta rule: an int8 query gives an fp16 attention_out
        _check(key.dtype == torch.int8 and value.dtype == torch.int8,
               "npu_fused_infer_attention_score: an int8 query takes an int8 key and value")
        return DT_FP16
    if kv8:
        _check(query.dtype in (torch.bfloat16, torch.float16) and value.dtype == torch.int8,
               "npu_fused_infer_attention_score: int8 key/value take a bf16 or fp16 query and an int8 value")
    else:
        _check(query.dtype in (torch.bfloat16, torch.float16) and key.dtype == query.dtype and
               value.dtype == query.dtype, "npu_fused_infer_attention_score: query/key/value must all be bf16 or all fp16")
    return DT_BF16 if query.dtype == torch.bfloat16 else DT_FP16


def _prefill_call(query, key, value, out, lse, want_lse, b, s_q, s_kv, hq, n_kv, d, dt, qs, ks, vs, os_, seq_q,
                  seq_kv, mask_origin, pre, nxt, bt, bs, kblk, vblk, scale, stream):
    _check(hq % n_kv == 0, "npu_fused_infer_attention_score: num_heads must be a multiple of num_key_value_heads")
    arr = [_ctypes_i64(qs), _ctypes_i64(ks), _ctypes_i64(vs), _ctypes_i64(os_)]
    ws_bytes = _lib.query("tai_fia_prefill_workspace_size", b, s_q, hq, n_kv)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=query.device)
    _lib.call("tai_fia_prefill", query.data_ptr(), key.data_ptr(), value.data_ptr(), b, s_q, s_kv, hq, n_kv, d, dt,
              arr[0], arr[1], arr[2], arr[3], seq_q.data_ptr() if seq_q is not None else None,
              seq_kv.data_ptr() if seq_kv is not None else None, mask_origin, pre, nxt,
              bt.data_ptr() if bt is not None else None, bt.size(1) if bt is not None else 0, bs, kblk, vblk, scale,
              out.data_ptr(), lse.data_ptr() if want_lse else None, ws.data_ptr(), ws_bytes, stream)
    return out, lse


def _ctypes_i64(vals):
    import ctypes
    return (ctypes.c_int64 * len(vals))(*vals)


def _mla(query, key, value, kw, out, lse, want_lse, num_heads, n_kv, bt, seq_kv, scale, stream):
    q_rope = kw["query_rope"]
    k_rope = kw.get("key_rope")
    k_scale = kw.get("key_antiquant_scale")
    _check(k_rope is not None, "npu_fused_infer_attention_score: MLA needs key_rope")
    _check(n_kv == 1, "npu_fused_infer_attention_score: MLA latent cache has one kv head")
    _check(key.dtype == torch.int8 and k_scale is not None and int(kw.get("key_antiquant_mode", 0)) == 1,
           "npu_fused_infer_attention_score: MLA serves an int8 latent cache with per-token scales "
           "(key_antiquant_mode=1)")
    _check(query.dtype == torch.bfloat16 and q_rope.dtype == torch.bfloat16 and k_rope.dtype == torch.bfloat16,
           "npu_fused_infer_attention_score: MLA query/query_rope/key_rope must be bf16")
    b = query.size(0)
    qn = query.contiguous()
    qr = q_rope.contiguous()
    dn = qn.numel() // (b * num_heads)
    dr = qr.numel() // (b * num_heads)
    kc = key.contiguous()
    nblk = kc.size(0)
    bs = kc.numel() // (nblk * dn)
    _check(kc.numel() == nblk * bs * dn, "npu_fused_infer_attention_score: latent cache must be [blocks, bs, 1, Dn]")
    kr = k_rope.contiguous()
    _check(kr.numel() == nblk * bs * dr, "npu_fused_infer_attention_score: key_rope must be [blocks, bs, 1, Dr]")
    ks = k_scale.to(torch.float32).contiguous()
    _check(ks.numel() == nblk * bs, "npu_fused_infer_attention_score: key_antiquant_scale must hold one fp32 per "
                                    "cached token ([blocks, bs])")
    ws_bytes = _lib.query("tai_fia_mla_decode_workspace_size", b, num_heads, dn, bt.size(1), bs)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=qn.device)
    _lib.call("tai_fia_mla_decode", qn.data_ptr(), qr.data_ptr(), kc.data_ptr(), ks.data_ptr(), kr.data_ptr(),
              bt.data_ptr(), bt.size(1), seq_kv.data_ptr(), b, num_heads, dn, dr, bs, scale, out.data_ptr(),
              lse.data_ptr() if want_lse else None, ws.data_ptr(), ws_bytes, stream)
    return out, lse


# ============================================================================ npu_fused_infer_attention_score_v2
# python/torchair/ops/_npu_fused_infer_attention_score_v2.py:14-30 (air:: schema, tensor lengths) and
# .../custom/fused_infer_attention_score_v2.py:14-60 (npu::, list or tensor lengths): the same operator
# under renamed arguments, lowered to the same FusedInferAttentionScore node (:166-181), so it maps onto
# the v1 implementation argument for argument. Arguments of v2 with no v1 counterpart that this build
# does not serve (query quantisation, the softmax quant scale, dtype reinterpretations) are refused;
# learnable_sink is passed on to the v1 implementation, which serves it on the general kernel.
_V2_UNSUPPORTED = ("dequant_scale_query", "quant_scale_p", "query_dtype", "key_dtype", "value_dtype",
                   "query_rope_dtype", "key_rope_dtype", "key_shared_prefix_dtype", "value_shared_prefix_dtype",
                   "dequant_scale_query_dtype", "dequant_scale_key_dtype", "dequant_scale_value_dtype",
                   "dequant_scale_key_rope_dtype")


def _v2_to_v1(kw: dict, check: bool = True) -> dict:
    name = "npu_fused_infer_attention_score_v2"
    if check:
        for k in _V2_UNSUPPORTED:
            _check(kw.get(k) is None, f"{name}: {k} is not supported")
        _check(kw.get("query_quant_mode", 0) == 0, f"{name}: query_quant_mode must be 0")
    m = {"pse_shift": "pse_shift", "atten_mask": "atten_mask", "actual_seq_qlen": "actual_seq_lengths",
         "actual_seq_kvlen": "actual_seq_lengths_kv", "block_table": "block_table",
         "dequant_scale_key": "key_antiquant_scale", "dequant_offset_key": "key_antiquant_offset",
         "dequant_scale_value": "value_antiquant_scale", "dequant_offset_value": "value_antiquant_offset",
         "dequant_scale_key_rope": "key_rope_antiquant_scale", "quant_scale_out": "quant_scale2",
         "quant_offset_out": "quant_offset2", "query_rope": "query_rope", "key_rope": "key_rope",
         "num_query_heads": "num_heads", "num_key_value_heads": "num_key_value_heads", "softmax_scale": "scale",
         "pre_tokens": "pre_tokens", "next_tokens": "next_tokens", "input_layout": "input_layout",
         "sparse_mode": "sparse_mode", "block_size": "block_size", "inner_precise": "inner_precise",
         "key_quant_mode": "key_antiquant_mode", "value_quant_mode": "value_antiquant_mode",
         "return_softmax_lse": "softmax_lse_flag", "learnable_sink": "learnable_sink"}
    return {m[k]: v for k, v in kw.items() if k in m}


def _v2_out_dtype(kw: dict, query):
    """attention_out dtype of the v2 meta rule (_npu_fused_infer_attention_score_v2.py:396-412): int8 (or
    out_dtype) with quant_scale_out, else the query dtype (int8 / fp8 queries are not served)."""
    od = kw.get("out_dtype")
    if kw.get("quant_scale_out") is not None:
        if od is None:
            return torch.int8
        from ._ops_impl import dtype_of_code, scalar_type_code
        return dtype_of_code(scalar_type_code(od))
    _check(od is None or od in (query.dtype, _torch_code(query.dtype)),
           "npu_fused_infer_attention_score_v2: out_dtype applies with quant_scale_out")
    return query.dtype


def _torch_code(dt):
    from ._ops_impl import scalar_type_code
    return scalar_type_code(dt)


def fia_v2_fake(query, key, value, **kw):
    out, lse = fia_fake(query, key, value, **_v2_to_v1(kw, check=False))
    od = _v2_out_dtype(kw, query)
    return (out if out.dtype == od else out.new_empty(out.shape, dtype=od)), lse


def fia_v2_cuda(query, key, value, **kw):
    """ROCm implementation of npu_fused_infer_attention_score_v2: the v1 kernels under the v1 names."""
    od = _v2_out_dtype(kw, query)
    out, lse = fia_cuda(query, key, value, **_v2_to_v1(kw))
    _check(out.dtype == od, "npu_fused_infer_attention_score_v2: out_dtype does not match the served output")
    return out, lse

