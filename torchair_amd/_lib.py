"""ctypes binding of libtai_kernels.so (the C ABI declared in include/tai_kernels.h).

The library is loaded lazily on the first kernel call. A missing or stale library is an
error: there is no fallback implementation behind these entry points.
"""
from __future__ import annotations

import ctypes
import threading
from ctypes import c_char_p, c_float, c_int, c_int64, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libtai_kernels.so"

# torch ScalarType codes used as dtype tags across the C ABI
DT_UINT8, DT_INT8, DT_INT16, DT_INT32, DT_INT64, DT_FP16, DT_FP32, DT_BF16 = 0, 1, 2, 3, 4, 5, 6, 15
DT_NONE = -1
LAYOUT_KN, LAYOUT_NK, LAYOUT_KN_SWIGLU = 0, 1, 2

_P = c_void_p
_I64x3 = c_int64 * 3


class FiaGeneralArgs(ctypes.Structure):
    """tai_fia_general_args (include/tai_kernels.h)."""
    _fields_ = [("dtype", c_int), ("dk1", c_int), ("dk2", c_int), ("dv", c_int),
                ("b", c_int64), ("s_q", c_int64), ("s_kv", c_int64), ("hq", c_int64), ("hkv", c_int64),
                ("q1", _P), ("q1_strides", _I64x3), ("q2", _P), ("q2_strides", _I64x3),
                ("k1", _P), ("k1_strides", _I64x3), ("k2", _P), ("k2_strides", _I64x3),
                ("v", _P), ("v_strides", _I64x3),
                ("block_table", _P), ("max_blocks", c_int64), ("block_size", c_int64),
                ("seq_lens_q", _P), ("seq_lens_kv", _P),
                ("mask", _P), ("mask_strides", _I64x3), ("mask_origin", c_int64),
                ("pre_tokens", c_int64), ("next_tokens", c_int64), ("scale", c_float),
                ("out", _P), ("out_strides", _I64x3), ("lse", _P),
                ("kv_dtype", c_int64), ("k_scale", _P), ("k_offset", _P), ("k_quant_mode", c_int64),
                ("v_scale", _P), ("v_offset", _P), ("v_quant_mode", c_int64), ("tok_stride", c_int64),
                ("out_dtype", c_int64), ("out_scale", _P), ("out_offset", _P), ("out_scale_len", c_int64),
                ("pse", _P), ("pse_strides", c_int64 * 4),
                ("k_prefix", _P), ("v_prefix", _P), ("k_prefix_strides", c_int64 * 2),
                ("v_prefix_strides", c_int64 * 2), ("prefix_len", _P), ("prefix_cap", c_int64),
                ("q_cum", _P), ("kv_cum", _P), ("q_dtype", c_int64), ("deq_scale1", _P), ("quant_scale1", _P),
                ("deq_scale2", _P), ("sink", _P)]


_SIGS = {
    "tai_last_error": (c_char_p, []),
    "tai_abi_version": (c_int, []),
    "tai_build_id": (c_char_p, []),
    "tai_calib_read_stream": (c_int, [_P, c_size_t, _P, c_size_t, _P]),
    "tai_dynamic_quant": (c_int, [_P, c_int, c_int64, c_int64, _P, _P, c_int, c_int64, _P, _P, _P]),
    "tai_dequant_swiglu_quant": (
        c_int, [_P, c_int64, c_int64, _P, _P, _P, c_int, _P, _P, c_int, c_int64, c_int, _P, _P, _P]),
    "tai_dequant_swiglu_quant_static": (
        c_int, [_P, c_int64, c_int64, _P, _P, _P, c_int, _P, _P, _P, c_int, c_int64, c_int, c_int, _P, _P, _P]),
    "tai_dequant_swiglu_quant_clamped": (
        c_int, [_P, c_int64, c_int64, _P, _P, _P, c_int, _P, _P, _P, c_int, c_int64, c_int, c_int, c_float, c_float,
                c_float, _P, _P, _P]),
    "tai_dynamic_quant_v2_workspace_size": (c_size_t, [c_int64]),
    "tai_dynamic_quant_v2": (
        c_int, [_P, c_int, c_int64, c_int64, _P, _P, c_int, c_int64, c_int, c_int, c_float, _P, _P, _P, _P, c_size_t,
                _P]),
    "tai_transpose_kn_to_nk": (c_int, [_P, c_int64, c_int64, _P, _P]),
    "tai_quant_matmul_prepack_wanted": (c_int, [c_int64, c_int64, c_int64]),
    "tai_quant_matmul_workspace_size": (c_size_t, [c_int64, c_int64, c_int64, c_int]),
    "tai_quant_matmul": (
        c_int, [_P, _P, c_int64, c_int64, c_int64, c_int, _P, c_int64, _P, c_int64, _P, _P, c_int, c_int, _P, _P,
                c_size_t, _P]),
    "tai_grouped_matmul_workspace_size": (c_size_t, [c_int64, c_int64, c_int64]),
    "tai_grouped_matmul": (
        c_int, [_P, _P, c_int64, c_int64, c_int64, c_int64, c_int, _P, c_int, _P, _P, _P, c_int, c_int, _P,
                _P, c_size_t, _P]),
    "tai_grouped_matmul_gather": (
        c_int, [_P, c_int64, _P, _P, c_int64, c_int64, c_int64, c_int64, c_int, _P, c_int, _P, _P, _P, c_int, c_int,
                _P, _P, c_size_t, _P]),
    "tai_grouped_matmul_noalloc_max_scratch": (c_size_t, []),
    "tai_grouped_matmul_noalloc": (
        c_int, [_P, _P, c_int64, c_int64, c_int64, c_int64, c_int, _P, c_int, _P, _P, _P, c_int, c_int, _P, _P]),
    "tai_grouped_matmul_swiglu_quant_workspace_size": (c_size_t, [c_int64, c_int64, c_int64]),
    "tai_swiglu_pack_kn": (c_int, [_P, c_int64, c_int64, _P, _P]),
    "tai_swiglu": (c_int, [_P, c_int, c_int64, c_int64, c_int64, _P, _P]),
    "tai_moe_compute_expert_tokens": (c_int, [_P, c_int64, c_int64, _P, _P]),
    "tai_grouped_matmul_swiglu_quant_gather": (
        c_int, [_P, c_int64, _P, _P, c_int64, c_int64, c_int64, c_int64, c_int, _P, c_int, _P, _P, _P, _P, _P, c_size_t,
                _P]),
    "tai_grouped_matmul_swiglu_quant": (
        c_int, [_P, _P, c_int64, c_int64, c_int64, c_int64, c_int, _P, c_int, _P, _P, _P, _P, _P, c_size_t, _P]),
    "tai_grouped_matmul_finalize_routing_workspace_size": (c_size_t, [c_int64, c_int64, c_int64, c_int64]),
    "tai_grouped_matmul_finalize_routing": (
        c_int, [_P, _P, c_int64, c_int64, c_int64, c_int64, c_int, _P, c_int, _P, _P, _P, _P, _P, c_int, _P, c_int64,
                c_float, c_int64, c_int64, _P, _P, c_size_t, _P]),
    "tai_moe_gating_top_k": (
        c_int, [_P, c_int, c_int64, c_int64, c_int, _P, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                c_float, c_float, _P, _P, _P, _P]),
    "tai_moe_init_routing_workspace_size": (c_size_t, [c_int64, c_int, c_int64]),
    "tai_moe_init_routing_v2_droppad_workspace_size": (c_size_t, [c_int64, c_int, c_int64, c_int64]),
    "tai_moe_init_routing_v2_droppad": (
        c_int, [_P, c_int, c_int64, c_int64, _P, c_int, _P, c_int64, c_int, c_int, c_int, _P, _P, _P, _P, _P, c_size_t,
                _P]),
    "tai_static_quant_rows": (
        c_int, [_P, c_int, c_int64, c_int64, _P, _P, c_int64, c_int, _P, c_int, c_int64, c_int64, _P, _P]),
    "tai_moe_init_routing_v2": (
        c_int, [_P, c_int, c_int64, c_int64, _P, c_int, _P, c_int64, c_int, c_int, c_int, c_int, _P, _P, _P,
                _P, _P, c_size_t, _P]),
    "tai_moe_init_routing_v2_rows": (
        c_int, [c_int64, _P, c_int, _P, c_int64, c_int, c_int, c_int, c_int, _P, _P, _P, _P, _P, c_size_t, _P]),
    "tai_moe_init_routing": (
        c_int, [_P, c_int, c_int64, c_int64, _P, _P, c_int, c_int64, c_int64, _P, _P, _P, _P, c_size_t, _P]),
    "tai_moe_finalize_routing": (
        c_int, [_P, c_int, c_int64, c_int64, c_int, _P, _P, _P, _P, c_int, _P, _P, c_int, _P, _P]),
    "tai_fia_paged_decode_workspace_size": (c_size_t, [c_int64, c_int, c_int, c_int64, c_int]),
    "tai_fia_paged_decode": (
        c_int, [_P, _P, _P, c_int64, c_int64, c_int64, _P, c_int64, _P, c_int64, c_int, c_int, c_int, c_int, c_int,
                c_float, _P, _P, _P, c_size_t, _P]),
    "tai_fia_paged_decode_sink": (
        c_int, [_P, _P, _P, c_int64, c_int64, c_int64, _P, c_int64, _P, c_int64, c_int, c_int, c_int, c_int, c_int,
                c_float, _P, _P, _P, _P, c_size_t, _P]),
    "tai_fia_paged_decode_kv8_workspace_size": (c_size_t, [c_int64, c_int, c_int, c_int, c_int64, c_int]),
    "tai_fia_paged_decode_kv8": (
        c_int, [_P, _P, _P, c_int64, c_int64, c_int64, _P, c_int64, _P, c_int64, c_int, c_int, c_int, c_int, c_int,
                c_float, _P, _P, _P, _P, _P, c_size_t, _P]),
    "tai_fia_prefill_workspace_size": (c_size_t, [c_int64, c_int64, c_int, c_int]),
    "tai_fia_prefill": (
        c_int, [_P, _P, _P, c_int64, c_int64, c_int64, c_int, c_int, c_int, c_int, _P, _P, _P, _P, _P, _P, c_int,
                c_int64, c_int64, _P, c_int64, c_int, c_int64, c_int64, c_float, _P, _P, _P, c_size_t, _P]),
    "tai_add_rms_norm": (c_int, [_P, _P, _P, c_int, c_int64, c_int64, c_float, _P, _P, _P, _P]),
    "tai_add_rms_norm_dynamic_quant": (
        c_int, [_P, _P, _P, _P, _P, _P, c_int, c_int64, c_int64, c_float, _P, _P, _P, _P, _P, _P]),
    "tai_scatter_pa_kv_cache": (
        c_int, [_P, _P, _P, _P, _P, c_int, c_int64, c_int64, c_int64, c_int64, c_int64, c_int, _P]),
    "tai_kv_rmsnorm_rope_cache": (
        c_int, [_P, _P, _P, _P, _P, c_int, c_int64, c_int64, c_int, c_int, c_float, _P, c_int, _P, c_int, c_int64,
                c_int64, _P, _P, _P, _P, _P, _P, _P, _P]),
    "tai_fia_general": (c_int, [ctypes.POINTER(FiaGeneralArgs), _P]),
    "tai_fia_general_args_size": (c_size_t, []),
    "tai_fia_mla_decode_workspace_size": (c_size_t, [c_int64, c_int, c_int, c_int64, c_int]),
    "tai_fia_mla_decode": (
        c_int, [_P, _P, _P, _P, _P, _P, c_int64, _P, c_int64, c_int, c_int, c_int, c_int, c_float, _P, _P, _P,
                c_size_t, _P]),
}

_lock = threading.Lock()
_lib = None


def exported_symbols():
    """Names of every entry point the header declares."""
    return list(_SIGS)


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                    "(hipcc --offload-arch=gfx950). The fused npu ops have no other implementation.")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in _SIGS.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _check_fresh(lib)
            if lib.tai_fia_general_args_size() != ctypes.sizeof(FiaGeneralArgs):
                raise RuntimeError(
                    f"{LIB_PATH}: tai_fia_general_args is {lib.tai_fia_general_args_size()} bytes in the library, "
                    f"{ctypes.sizeof(FiaGeneralArgs)} in _lib.FiaGeneralArgs; the two layouts differ")
            _lib = lib
    return _lib


def _check_fresh(lib: ctypes.CDLL) -> None:
    """Refuses a library built from other sources than the ones beside it."""
    from . import _build
    if not _build.CSRC.is_dir():  # an installed copy without sources: nothing to compare against
        return
    want = _build.source_id()
    got = lib.tai_build_id().decode(errors="replace")
    if got != want:
        raise RuntimeError(
            f"{LIB_PATH} is stale: built from sources {got}, the sources beside it hash to {want}; rebuild "
            "with `python -c 'import __graft_entry__ as g; g.build()'`")


class KernelError(RuntimeError):
    pass


def call(name: str, *args) -> None:
    """Calls a status-returning entry point; raises RuntimeError with the library's message."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.tai_last_error().decode(errors="replace")
        raise KernelError(f"{name} failed (status {rc}): {msg}")


def query(name: str, *args) -> int:
    return int(getattr(load(), name)(*args))
