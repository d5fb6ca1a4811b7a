"""Seeded input generators and comparison helpers shared by the tests."""
from __future__ import annotations

import numpy as np
import torch


def gen(seed: int = 0) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def randn(shape, g, dtype=torch.bfloat16):
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype)


def rand_i8(shape, g):
    return torch.randint(-127, 128, shape, generator=g, dtype=torch.int8)


def uniform(shape, g, lo, hi):
    return torch.rand(shape, generator=g, dtype=torch.float32) * (hi - lo) + lo


def f32np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def assert_int8_close(got: np.ndarray, want: np.ndarray, max_frac: float = 1e-3):
    """int8 outputs within +-1 LSB, with at most max_frac of elements differing."""
    got = got.astype(np.int32)
    want = want.astype(np.int32)
    diff = np.abs(got - want)
    assert diff.max(initial=0) <= 1, f"int8 differs by {diff.max()} LSB"
    frac = float((diff > 0).mean()) if diff.size else 0.0
    assert frac <= max_frac, f"{frac:.2e} of int8 elements differ (limit {max_frac})"


def assert_close(got, want, rtol=1e-2, atol=1e-2):
    np.testing.assert_allclose(np.asarray(got, np.float32), np.asarray(want, np.float32), rtol=rtol, atol=atol)
