"""GPU: every case a converter declares with declare_supported runs eagerly and compiled through
get_npu_backend (hipGraph capture), and the two agree bit for bit; both also match the CPU oracle.
This is the reference's converter smoke test (tests/smoke/converter_test.py:150-247, which runs
each declared case eager vs graph) on this backend. Floating inputs are seeded random values of
the declared shape and dtype; integer inputs are the declared values (index tensors)."""
import numpy as np
import pytest
import torch

import torchair_amd
from torchair_amd.converter import declared_supported_converters
from tests.helpers import assert_close, assert_int8_close

DEV = "cuda"
_CASES = [(op, i) for op, conv in declared_supported_converters().items() for i in range(len(conv.supported_cases))]


def _materialize(v, g):
    if isinstance(v, torch.Tensor):
        if v.dtype.is_floating_point:
            return torch.randn(v.shape, generator=g).to(v.dtype)
        return v.clone()
    if isinstance(v, (list, tuple)):
        return type(v)(_materialize(x, g) for x in v)
    if isinstance(v, dict):
        return {k: _materialize(x, g) for k, x in v.items()}
    return v


def _to(v, dev):
    if isinstance(v, torch.Tensor):
        return v.to(dev)
    if isinstance(v, (list, tuple)):
        return type(v)(_to(x, dev) for x in v)
    if isinstance(v, dict):
        return {k: _to(x, dev) for k, x in v.items()}
    return v


def _flat(out):
    if isinstance(out, torch.Tensor):
        return [out]
    return [t for t in out if isinstance(t, torch.Tensor)]


@pytest.mark.gpu
@pytest.mark.parametrize("op,idx", _CASES, ids=[f"{op}-{i}" for op, i in _CASES])
def test_declared_case_eager_equals_compiled_and_oracle(op, idx):
    from oracle import cpu_ops
    cpu_ops.register()
    torch._dynamo.reset()  # one lambda code object serves every case: start each from a clean cache
    case = declared_supported_converters()[op].supported_cases[idx]
    g = torch.Generator().manual_seed(1000 + idx)
    args = _materialize(case.args, g)
    kwargs = _materialize(case.kwargs, g)
    dargs, dkw = _to(args, DEV), _to(kwargs, DEV)
    eager = _flat(op(*dargs, **dkw))
    cfg = torchair_amd.CompilerConfig()
    cfg.mode = "reduce-overhead"
    fn = torch.compile(lambda *a: op(*a, **dkw), backend=torchair_amd.get_npu_backend(compiler_config=cfg),
                       fullgraph=True)
    for _ in range(2):  # capture, then a replay
        compiled = _flat(fn(*dargs))
        assert len(compiled) == len(eager)
        for a, b in zip(compiled, eager):
            assert a.dtype == b.dtype and a.shape == b.shape
            assert torch.equal(torch.nan_to_num(a.float(), 7.0), torch.nan_to_num(b.float(), 7.0))
    want = _flat(op(*args, **kwargs))  # the oracle's CPU kernels
    for got, w in zip(eager, want):
        got = got.cpu()
        if got.dtype == torch.int8:
            assert_int8_close(got.numpy(), w.numpy())
        elif not got.dtype.is_floating_point:
            np.testing.assert_array_equal(got.numpy(), w.numpy())
        else:
            assert_close(got.float().numpy(), w.float().numpy())
