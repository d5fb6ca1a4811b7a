"""Seeded random grouped W8A8 GEMMs, exact in int32 against an int64 product: group sizes on both sides
of every tile boundary (32, 64, 128 and 256 rows, empty groups), rows past the grouped total, N on and
off the mixed-tile path (multiples of 512 and not), [K, N] and [N, K] weights, cumulative and count
group lists; and the gathered form (tai::grouped_matmul_gather) on random row maps."""
import numpy as np
import pytest
import torch

import torchair_amd  # noqa: F401

pytestmark = pytest.mark.gpu
DEV = "cuda"
_EDGE = [0, 1, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 257, 300]


def _case(seed):
    rng = np.random.default_rng(3000 + seed)
    e = int(rng.integers(2, 10))
    counts = [int(rng.choice(_EDGE)) if rng.random() < 0.7 else int(rng.integers(0, 400)) for _ in range(e)]
    k = 64 * int(rng.integers(1, 20))
    n = int(rng.choice([512, 1024, 576, 256, 1536]))
    extra = int(rng.integers(0, 40))
    return rng, e, counts, k, n, extra


def _ref(x, w, counts):
    """int64 product, group by group; rows past the total are zero."""
    out = torch.zeros(x.shape[0], w.shape[2], dtype=torch.int64)
    b = 0
    for g, c in enumerate(counts):
        out[b:b + c] = x[b:b + c].long() @ w[g].long()
        b += c
    return out


@pytest.mark.parametrize("seed", range(12))
def test_random_grouped_matmul_int32(seed):
    rng, e, counts, k, n, extra = _case(seed)
    g = torch.Generator().manual_seed(3000 + seed)
    m = sum(counts) + extra
    x = torch.randint(-128, 128, (m, k), generator=g, dtype=torch.int8)
    w = torch.randint(-128, 128, (e, k, n), generator=g, dtype=torch.int8)
    nk = bool(rng.integers(0, 2))
    list_type = int(rng.integers(0, 2))
    gl = torch.tensor(counts if list_type == 1 else np.cumsum(counts).tolist(), dtype=torch.int64)
    wd = w.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) if nk else w.to(DEV)
    case = dict(e=e, counts=counts, k=k, n=n, extra=extra, nk=nk, list_type=list_type)
    print("case", case, flush=True)
    out = torch.ops.npu.npu_grouped_matmul([x.to(DEV)], [wd], group_list=gl.to(DEV), split_item=3, group_type=0,
                                           group_list_type=list_type, output_dtype=torch.int32)[0]
    assert torch.equal(out.cpu().long(), _ref(x, w, counts)), case


@pytest.mark.parametrize("seed", range(6))
def test_random_grouped_matmul_gather(seed):
    rng, e, counts, k, n, _ = _case(seed)
    g = torch.Generator().manual_seed(3100 + seed)
    t = int(rng.integers(1, 200))
    m = sum(counts)
    x = torch.randint(-128, 128, (t, k), generator=g, dtype=torch.int8)
    w = torch.randint(-128, 128, (e, k, n), generator=g, dtype=torch.int8)
    a_rows = torch.randint(0, t, (m,), generator=g, dtype=torch.int32)
    gl = torch.tensor(counts, dtype=torch.int64)
    case = dict(e=e, counts=counts, k=k, n=n, t=t)
    print("case", case, flush=True)
    out = torch.ops.tai.grouped_matmul_gather(x.to(DEV), a_rows.to(DEV), w.to(DEV), gl.to(DEV), group_list_type=1,
                                              output_dtype=torch.int32)
    assert torch.equal(out.cpu().long(), _ref(x[a_rows.long()], w, counts)), case
