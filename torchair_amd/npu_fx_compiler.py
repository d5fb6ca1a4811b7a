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
import operator
from typing import Any, Callable, Dict, List, Optional

import torch
import torch.fx

from . import converters as _converters  # noqa: F401  (registers the hot-path converters)
from .configs import CompilerConfig, check_config_support
from .converter import _get_converter
from . import graph as _graph
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


def _placeholder_index(gm: torch.fx.GraphModule) -> Dict[torch.fx.Node, int]:
    return {n: i for i, n in enumerate(n for n in gm.graph.nodes if n.op == "placeholder")}


def reinplace_mutations(gm: torch.fx.GraphModule) -> int:
    """Turns ``auto_functionalized_v2(op, ..., _all_bases=[cache, ...])`` whose results are only copied
    back into graph inputs (``aten.copy_(cache, getitem)``) into the in-place ``op`` on those inputs.

    This is the re-inplacing the reference registers for its in-place cache writers
    (python/torchair/_acl_concrete_graph/graph_pass.py:160-163): without it every call clones the KV
    cache and copies it back. A base is re-inplaced only when it is a graph input that is the
    mutable argument itself (not a view of it) and nothing after the call reads its old value."""
    hop = getattr(torch.ops.higher_order, "auto_functionalized_v2", None)
    if hop is None:
        return 0
    order = {n: i for i, n in enumerate(gm.graph.nodes)}
    done = 0
    for node in list(gm.graph.nodes):
        if node.op != "call_function" or node.target is not hop:
            continue
        op = node.args[0]
        kw = dict(node.kwargs)
        bases = kw.pop("_all_bases", [])
        mutable = [a.name for a in op._schema.arguments if a.alias_info is not None and a.alias_info.is_write]
        getitems = {}
        ok = all(u.op == "call_function" and u.target is operator.getitem for u in node.users)
        for u in node.users if ok else ():
            getitems.setdefault(u.args[1], []).append(u)
        new_kwargs = {}
        copies = []
        for name in mutable:
            bi = kw.pop(f"_{name}_base_index", None)
            if bi is None or any(f"_{name}_{t}" in kw for t in ("size", "stride", "storage_offset", "slice_dim")):
                ok = False
                break
            base = bases[bi]
            if not isinstance(base, torch.fx.Node) or base.op != "placeholder":
                ok = False
                break
            for gi in getitems.get(bi + 1, []):
                for cu in gi.users:
                    if cu.target is torch.ops.aten.copy_.default and cu.args[0] is base and cu.args[1] is gi:
                        copies.append(cu)
                    else:
                        ok = False
            later = [u for u in base.users if u is not node and u not in copies and order[u] > order[node]]
            if later:
                ok = False
            new_kwargs[name] = base
        if not ok or any(k.startswith("_") for k in kw):
            continue
        new_kwargs.update(kw)
        with gm.graph.inserting_before(node):
            call = gm.graph.call_function(op, (), new_kwargs)
        for cu in copies:
            gm.graph.erase_node(cu)
        for idx, users in getitems.items():
            for gi in users:
                if idx == 0:
                    gi.replace_all_uses_with(call)
                if not gi.users:
                    gm.graph.erase_node(gi)
        if not node.users:
            gm.graph.erase_node(node)
            done += 1
    if done:
        gm.graph.lint()
        gm.recompile()
    return done


def mutated_inputs(gm: torch.fx.GraphModule) -> List[int]:
    """Positions of the graph inputs that the graph writes in place: arguments marked mutable
    (``Tensor(a!)``) in the schema of a call, and destinations of ``aten.copy_``."""
    ph = _placeholder_index(gm)
    out = set()
    for n in gm.graph.nodes:
        if n.op != "call_function":
            continue
        schema = getattr(n.target, "_schema", None)
        if schema is None:
            continue
        for i, a in enumerate(schema.arguments):
            if a.alias_info is None or not a.alias_info.is_write:
                continue
            v = n.args[i] if i < len(n.args) else n.kwargs.get(a.name)
            for t in (v if isinstance(v, (list, tuple)) else [v]):
                if isinstance(t, torch.fx.Node) and t in ph:
                    out.add(ph[t])
    return sorted(out)


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
        reinplace_mutations(gm)
        lowered = lower_graph(gm)
        if self.config.debug.run_eagerly.value:
            return lowered
        dbg = self.config.debug.aclgraph
        runner = HipGraphRunner(lowered, capture_limit=dbg.static_capture_size_limit.value,
                                clone_output=bool(dbg.enable_output_clone.value),
                                clone_input=bool(dbg.clone_input.value), mutated_inputs=mutated_inputs(lowered))
        runner.lowered = lowered
        return _safe_runner(runner, lowered)


def _safe_runner(runner: HipGraphRunner, eager: Callable) -> Callable:
    """Captures on the first call per signature; a graph that cannot be captured runs eagerly."""
    state = {"broken": False}

    def run(*args):
        if state["broken"]:
            _graph.stats["eager_fallbacks"] += 1
            return eager(*args)
        try:
            return runner(*args)
        except RuntimeError as e:
            if "captur" not in str(e).lower() and "graph" not in str(e).lower():
                raise
            logger.warning("hipGraph capture failed (%s); running the lowered graph eagerly", e)
            state["broken"] = True
            _graph.stats["eager_fallbacks"] += 1
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
