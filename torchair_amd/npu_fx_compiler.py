"""Dynamo backend: ``get_npu_backend(compiler_config=...)``.

Call path (reference: python/torchair/npu_fx_compiler.py:865-1005):
  torch.compile -> _npu_backend(gm, example_inputs) -> aot_module_simplified(fw_compiler=_NpuFxCompiler)
  -> _NpuFxCompiler(gm): every FX node whose target has a registered converter is replaced by
     what the converter emits (the fused npu ops lower onto the torch.library ops served by
     libtai_kernels.so; other aten ops stay for PyTorch-ROCm), then the lowered module is
     wrapped in a HipGraphRunner (capture per input signature, replay afterwards) unless
     ``debug.run_eagerly`` is set.
"""
from __future__ import annotations

import functools
import logging
from typing import Any, Callable, Dict, List, Optional

import torch
import torch.fx

from . import converters as _converters  # noqa: F401  (registers the hot-path converters)
from .configs import CompilerConfig, check_config_support
from .converter import _get_converter
from .graph import HipGraphRunner
from .patterns import apply_pattern_passes

logger = logging.getLogger("torchair_amd")


class _NpuGraphConverter(torch.fx.Transformer):
    """Rebuilds an FX graph, replacing nodes that have a converter by the converter's output."""

    def run_node(self, n: torch.fx.Node):
        self._node = n
        return super().run_node(n)

    def call_function(self, target, args, kwargs):
        conv = _get_converter(target)
        if conv is None:
            return super().call_function(target, args, kwargs)
        meta = self._node.meta.get("val") if self._node is not None else None
        return conv(*args, meta_outputs=meta, **kwargs)


def lower_graph(gm: torch.fx.GraphModule) -> torch.fx.GraphModule:
    lowered = _NpuGraphConverter(gm).transform()
    lowered.graph.eliminate_dead_code()
    lowered.recompile()
    return lowered


class _NpuFxCompiler:
    def __init__(self, compiler_config: CompilerConfig):
        self.config = compiler_config

    def __call__(self, gm: torch.fx.GraphModule, example_inputs: List[Any]):
        # pattern passes run on the aten/npu graph, as in python/torchair/npu_fx_compiler.py:337-338
        if self.config.experimental_config.pattern_fusion_pass.value:
            apply_pattern_passes(gm)
        lowered = lower_graph(gm)
        if self.config.debug.run_eagerly.value:
            return lowered
        dbg = self.config.debug.aclgraph
        runner = HipGraphRunner(lowered, capture_limit=dbg.static_capture_size_limit.value,
                                clone_output=bool(dbg.enable_output_clone.value),
                                clone_input=bool(dbg.clone_input.value))
        runner.lowered = lowered
        return _safe_runner(runner, lowered)


def _safe_runner(runner: HipGraphRunner, eager: Callable) -> Callable:
    """Captures on the first call per signature; a graph that cannot be captured runs eagerly."""
    state = {"broken": False}

    def run(*args):
        if state["broken"]:
            return eager(*args)
        try:
            return runner(*args)
        except RuntimeError as e:
            if "captur" not in str(e).lower() and "graph" not in str(e).lower():
                raise
            logger.warning("hipGraph capture failed (%s); running the lowered graph eagerly", e)
            state["broken"] = True
            return eager(*args)

    run.runner = runner
    return run


def get_compiler(compiler_config: Optional[CompilerConfig] = None) -> _NpuFxCompiler:
    return _NpuFxCompiler(compiler_config or CompilerConfig())


def _npu_backend(gm: torch.fx.GraphModule, example_inputs: List[Any], compiler_config: CompilerConfig = None,
                 decompositions: Optional[Dict] = None, **kwargs):
    from torch._functorch.aot_autograd import aot_module_simplified
    compiler = get_compiler(compiler_config)
    return aot_module_simplified(gm, example_inputs, fw_compiler=compiler, decompositions=decompositions or {},
                                 keep_inference_input_mutations=True)


def get_npu_backend(*, compiler_config: CompilerConfig = None, custom_decompositions: Dict = None):
    """Backend for ``torch.compile(model, backend=get_npu_backend(compiler_config=cfg))``."""
    if compiler_config is None:
        compiler_config = CompilerConfig()
    check_config_support(compiler_config)
    return functools.partial(_npu_backend, compiler_config=compiler_config,
                             decompositions=dict(custom_decompositions or {}))
