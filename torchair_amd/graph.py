"""hipGraph capture/replay of a lowered FX graph.

Plays the role of the reference's graph executors (GE session run,
torchair/npu_graph_executor/*, and the ACL graph capture of
python/torchair/_acl_concrete_graph/acl_graph.py:825-848, 1174-1288, 1290-1402):
one graph per input signature, inputs copied into graph-owned buffers before a replay,
parameters used in place. Sequence lengths, block tables and group lists are device
tensors read by the kernels, so a replay with new values needs no re-capture.
"""
from __future__ import annotations

import logging
from typing import Any, Callable, Dict, List, Sequence, Tuple

import torch

logger = logging.getLogger("torchair_amd")


def _signature(args: Sequence[Any]) -> Tuple:
    sig = []
    for a in args:
        if isinstance(a, torch.Tensor):
            sig.append(("T", tuple(a.shape), tuple(a.stride()), a.dtype, str(a.device)))
        else:
            sig.append(("V", a))
    return tuple(sig)


class _Captured:
    def __init__(self, fn: Callable, args: Sequence[Any], clone_input: bool):
        self.static_idx: List[int] = []
        self.inputs: List[Any] = []
        for i, a in enumerate(args):
            if isinstance(a, torch.Tensor) and (isinstance(a, torch.nn.Parameter) or not clone_input):
                self.static_idx.append(i)
                self.inputs.append(a)
            elif isinstance(a, torch.Tensor):
                self.inputs.append(a.clone())
            else:
                self.inputs.append(a)
        self.static_ptrs = {i: args[i].data_ptr() for i in self.static_idx}
        dev = next((a.device for a in args if isinstance(a, torch.Tensor)), torch.device("cuda"))
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            fn(*self.inputs)  # warm-up: allocator state and lazy library loading outside capture
        torch.cuda.current_stream(dev).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            out = fn(*self.inputs)
        self.outputs = out

    def run(self, args: Sequence[Any]):
        for i, a in enumerate(args):
            if not isinstance(a, torch.Tensor):
                continue
            if i in self.static_ptrs:
                if a.data_ptr() != self.static_ptrs[i]:
                    raise RuntimeError("a static (parameter) input changed its storage after capture; "
                                       "recompile or set debug.aclgraph.clone_input=True")
                continue
            self.inputs[i].copy_(a)
        self.graph.replay()
        return self.outputs


class HipGraphRunner:
    """Callable that captures ``fn`` per input signature and replays it."""

    def __init__(self, fn: Callable, capture_limit: int = 64, clone_output: bool = False,
                 clone_input: bool = True):
        self.fn = fn
        self.capture_limit = capture_limit
        self.clone_output = clone_output
        self.clone_input = clone_input
        self.graphs: Dict[Tuple, _Captured] = {}
        self._warned = False

    def __call__(self, *args):
        if not any(isinstance(a, torch.Tensor) and a.is_cuda for a in args):
            return self.fn(*args)
        key = _signature(args)
        entry = self.graphs.get(key)
        if entry is None:
            if len(self.graphs) >= self.capture_limit:
                if not self._warned:
                    logger.warning("static_capture_size_limit (%d) reached; running eagerly", self.capture_limit)
                    self._warned = True
                return self.fn(*args)
            entry = _Captured(self.fn, args, self.clone_input)
            self.graphs[key] = entry
        out = entry.run(args)
        if self.clone_output:
            out = _map_tensors(out, lambda t: t.clone())
        return out


def _map_tensors(obj, f):
    if isinstance(obj, torch.Tensor):
        return f(obj)
    if isinstance(obj, (list, tuple)):
        return type(obj)(_map_tensors(o, f) for o in obj)
    return obj
