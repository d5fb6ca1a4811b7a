"""hipGraph capture/replay of a lowered FX graph.

Plays the role of the reference's graph executors (GE session run,
torchair/npu_graph_executor/*, and the ACL graph capture of
python/torchair/_acl_concrete_graph/acl_graph.py:825-848, 1174-1288, 1290-1402):
one graph per input signature, inputs copied into graph-owned buffers before a replay,
parameters and inputs the graph writes in place (KV caches) used by pointer. Sequence lengths, block tables and group lists are device
tensors read by the kernels, so a replay with new values needs no re-capture.
"""
from __future__ import annotations

import logging
import threading
from typing import Any, Callable, Dict, List, Sequence, Tuple

import torch

logger = logging.getLogger("torchair_amd")

# process-wide counts, for diagnostics and tests: graphs captured, and calls that ran eagerly
# because a graph could not be captured or the capture limit was reached
stats = {"captures": 0, "eager_fallbacks": 0}

_state = threading.local()


def preparing_capture() -> bool:
    """True while the eager warm-up run that precedes a capture is executing (on this thread). Ops
    that need host-side resources inside the captured graph (pinned buffers) create them then:
    nothing may allocate pinned memory while a stream is being captured."""
    return getattr(_state, "warmup", False)


def capture_resources():
    """The dict of host-side resources owned by the graph being prepared or captured on this thread
    (None outside a capture). Ops keep what a captured graph reads at replay time (pinned buffers)
    there, so it lives exactly as long as that graph."""
    return getattr(_state, "resources", None)


def _signature(args: Sequence[Any], pinned: Sequence[bool]) -> Tuple:
    sig = []
    for a, pin in zip(args, pinned):
        if isinstance(a, torch.Tensor):
            # a parameter or an input the graph writes in place is part of the captured graph by its
            # address: another address captures anew, as the reference re-captures when a mutated
            # input or a parameter moves (acl_graph.py:1195, 1361-1372)
            sig.append(("T", tuple(a.shape), tuple(a.stride()), a.dtype, str(a.device), a.data_ptr() if pin else None))
        else:
            sig.append(("V", a))
    return tuple(sig)


class _Captured:
    """One captured graph. Inputs passed by pointer (parameters, inputs the graph writes in place,
    or every tensor when ``clone_input`` is off) are used as they are; the others are copied into
    graph-owned buffers before each replay. A by-pointer input that is neither a parameter nor
    written in place is retained at its capture-time address; a replay that passes another tensor
    there copies it into the retained one first (acl_graph.py:1329-1337)."""

    def __init__(self, fn: Callable, args: Sequence[Any], by_pointer: Sequence[bool], pinned: Sequence[bool]):
        self.copy_idx: List[int] = []
        self.moved_idx: List[Tuple[int, int]] = []
        self.inputs: List[Any] = []
        for i, (a, ptr, pin) in enumerate(zip(args, by_pointer, pinned)):
            if isinstance(a, torch.Tensor) and not ptr:
                self.copy_idx.append(i)
                self.inputs.append(a.clone())
            else:
                if isinstance(a, torch.Tensor) and not pin:
                    self.moved_idx.append((i, a.data_ptr()))
                self.inputs.append(a)
        dev = next((a.device for a in args if isinstance(a, torch.Tensor) and a.is_cuda), torch.device("cuda"))
        self.resources: Dict[Any, Any] = {}
        _state.resources = self.resources
        try:
            self._capture(fn, dev)
        finally:
            _state.resources = None
        stats["captures"] += 1

    def _capture(self, fn: Callable, dev: torch.device):
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            # warm-up outside capture (allocator state, lazy library loading); its result is the
            # result of this first call, so side effects on inputs happen exactly once per call
            _state.warmup = True
            try:
                self.first_outputs = fn(*self.inputs)
            finally:
                _state.warmup = False
        torch.cuda.current_stream(dev).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            out = fn(*self.inputs)
        self.outputs = out

    def run(self, args: Sequence[Any]):
        for i in self.copy_idx:
            self.inputs[i].copy_(args[i])
        for i, ptr in self.moved_idx:
            if args[i].data_ptr() != ptr:
                self.inputs[i].copy_(args[i])
        self.graph.replay()
        return self.outputs


class HipGraphRunner:
    """Callable that captures ``fn`` per input signature and replays it.

    ``mutated_inputs``: positions of the inputs ``fn`` writes in place (KV caches); they are never
    copied, so the caller's tensors see the writes."""

    def __init__(self, fn: Callable, capture_limit: int = 64, clone_output: bool = False,
                 clone_input: bool = True, mutated_inputs: Sequence[int] = ()):
        self.fn = fn
        self.capture_limit = capture_limit
        self.clone_output = clone_output
        self.clone_input = clone_input
        self.mutated_inputs = frozenset(mutated_inputs)
        self.graphs: Dict[Tuple, _Captured] = {}
        self._warned = False

    def _by_pointer(self, args) -> List[bool]:
        return [isinstance(a, torch.Tensor) and (not self.clone_input or isinstance(a, torch.nn.Parameter)
                                                 or i in self.mutated_inputs) for i, a in enumerate(args)]

    def _pinned(self, args) -> List[bool]:
        return [isinstance(a, torch.Tensor) and (isinstance(a, torch.nn.Parameter) or i in self.mutated_inputs)
                for i, a in enumerate(args)]

    def __call__(self, *args):
        if not any(isinstance(a, torch.Tensor) and a.is_cuda for a in args):
            return self.fn(*args)
        by_ptr = self._by_pointer(args)
        pinned = self._pinned(args)
        key = _signature(args, pinned)
        entry = self.graphs.get(key)
        if entry is None:
            if len(self.graphs) >= self.capture_limit:
                if not self._warned:
                    logger.warning("static_capture_size_limit (%d) reached; running eagerly", self.capture_limit)
                    self._warned = True
                stats["eager_fallbacks"] += 1
                return self.fn(*args)
            entry = _Captured(self.fn, args, by_ptr, pinned)
            self.graphs[key] = entry
            out = entry.first_outputs
            entry.first_outputs = None
        else:
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
