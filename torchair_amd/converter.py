"""Converter registry: the extension surface of
python/torchair/_ge_concrete_graph/fx2ge_converter.py:221-235 and :327-414.

``register_fx_node_ge_converter(op)`` returns a ``Converter``; decorating a function with it
attaches the wrapped function to the OpOverload as ``_ge_converter`` (or keeps it in a
module table when the attribute cannot be set). When the backend lowers an FX graph, a
converter is called with the node's arguments - FX proxies in the lowered graph - plus
``meta_outputs`` (the node's fake-tensor results) when its signature asks for it, and
whatever it returns replaces the node. Converters therefore lower a node by calling
ops (the fused ``torch.ops.npu.*`` ops, or any other torch op) on their arguments.
"""
from __future__ import annotations

import functools
import inspect
from typing import Any, Callable, Dict, List, Optional

_CONVERTERS: Dict[Any, Callable] = {}
_DECLARED_SUPPORTED_CONVERTERS: Dict[Any, "Converter"] = {}


class Support:
    """One declared test case: positional and keyword example inputs of a converter."""

    def __init__(self, *args, **kwargs):
        self.args = args
        self.kwargs = kwargs


def _wrap_converter(converter: Callable) -> Callable:
    wants_meta = "meta_outputs" in inspect.signature(converter).parameters

    @functools.wraps(converter)
    def wrapped(*args, meta_outputs=None, **kwargs):
        if wants_meta:
            kwargs["meta_outputs"] = meta_outputs
        return converter(*args, **kwargs)

    wrapped.require_meta = wants_meta
    return wrapped


class Converter:
    def __init__(self, aten_op) -> None:
        self._aten_op = aten_op
        try:
            self._signature = inspect.signature(aten_op)
        except (TypeError, ValueError):
            self._signature = None
        self._supported_cases: Optional[List[Support]] = None

    def __call__(self, converter: Callable) -> "Converter":
        wrapped = _wrap_converter(converter)
        try:
            self._aten_op._ge_converter = wrapped
        except Exception:
            _CONVERTERS[self._aten_op] = wrapped
        return self

    @property
    def supported_cases(self):
        return self._supported_cases

    @supported_cases.setter
    def supported_cases(self, cases):
        for c in cases:
            if not isinstance(c, Support):
                raise AssertionError(f"declared cases must be Support objects, got {type(c).__name__}")
        self._supported_cases = cases


def declare_supported(supported_cases: List[Support]):
    def add(converter):
        if not isinstance(converter, Converter):
            raise AssertionError("declare_supported decorates what register_fx_node_ge_converter returned")
        converter.supported_cases = supported_cases
        _DECLARED_SUPPORTED_CONVERTERS[converter._aten_op] = converter
        return converter
    return add


def _empty_function(*args, **kwargs):
    pass


def register_fx_node_ge_converter(aten_op):
    """Registers a converter for a torch operation; None returns a no-op decorator."""
    if aten_op is None:
        return _empty_function
    return Converter(aten_op)


def _get_converter(target) -> Optional[Callable]:
    if target in _CONVERTERS:
        return _CONVERTERS[target]
    return getattr(target, "_ge_converter", None)


def declared_supported_converters():
    return dict(_DECLARED_SUPPORTED_CONVERTERS)
