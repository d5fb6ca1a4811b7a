"""torchair_amd: the TorchAir graph-mode API on AMD Instinct MI355X (gfx950).

Public surface kept from python/torchair/__init__.py:1-50: ``get_npu_backend``,
``get_compiler``, ``CompilerConfig``, ``register_fx_node_ge_converter``, ``ops``, ``logger``.
The fused npu ops are ``torch.library`` ops served by hand-written HIP kernels in
``libtai_kernels.so``.
"""
import logging

from . import _ops_impl  # noqa: F401  (defines torch.ops.npu / npu_inference / air ops)
from . import ops  # noqa: F401
from .configs import CompilerConfig
from .converter import register_fx_node_ge_converter
from .npu_fx_compiler import get_compiler, get_npu_backend

logger = logging.getLogger("torchair_amd")

__all__ = ["get_compiler", "get_npu_backend", "CompilerConfig", "register_fx_node_ge_converter", "logger", "ops"]
