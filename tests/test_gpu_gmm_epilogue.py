"""GPU parity: grouped GEMMs over skewed group lists, exact. Edge cases: K of exactly four 64-byte stages,
empty groups, groups of one row tile (non-temporal weight loads), rows past the grouped total (zero fill),
both weight layouts and every output dtype. Integer outputs are compared exactly with a float64 product;
floating outputs bit for bit with the op's fp32 arithmetic ((acc * scale) * per_token_scale, rounded to
fp32 and then to the output type, nearest even)."""
import pytest
import torch

import torchair_amd  # noqa: F401

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(seed, e, k, n, counts, extra_rows=0):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    counts = torch.tensor(counts, dtype=torch.int64, device=DEV)
    m = int(counts.sum()) + extra_rows
    x = torch.randint(-127, 128, (m, k), generator=g, device=DEV, dtype=torch.int8)
    w = torch.randint(-127, 128, (e, k, n), generator=g, device=DEV, dtype=torch.int8)
    return x, w, counts


def _exact(x, w, counts):
    """int64 product per group; rows past the grouped total are zero."""
    out = torch.zeros(x.shape[0], w.shape[2], dtype=torch.int64, device=DEV)
    b0 = 0
    for ei, c in enumerate(counts.tolist()):
        if c:
            out[b0:b0 + c] = torch.matmul(x[b0:b0 + c].double(), w[ei].double()).round().to(torch.int64)
        b0 += c
    return out


def _counts(e, seed):
    """Skewed row counts: empty groups, groups of one row tile, groups of many."""
    g = torch.Generator()
    g.manual_seed(seed)
    c = torch.randint(0, 900, (e,), generator=g)
    c[1] = 0
    c[4] = 1
    c[5] = 128
    c[6] = 129
    c[e - 1] = 0
    return c.tolist()


@pytest.mark.parametrize("layout,k", [("kn", 256), ("kn", 704), ("nk", 256), ("nk", 576)])
def test_grouped_int32_exact_skewed(layout, k):
    e, n = 16, 4096
    x, w, counts = _case(31, e, k, n, _counts(e, 31), extra_rows=300)
    wd = w if layout == "kn" else w.transpose(1, 2).contiguous().transpose(1, 2)
    out = torch.ops.npu.npu_grouped_matmul([x], [wd], group_list=counts, split_item=3, group_type=0,
                                           group_list_type=1, output_dtype=torch.int32)[0]
    want = _exact(x, w, counts)
    assert torch.equal(out.to(torch.int64), want)


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("with_pts", [True, False])
@pytest.mark.parametrize("big", [True, False])
def test_grouped_float_epilogue_bitexact(out_dtype, with_pts, big):
    e, k, n = (16, 512, 3584) if big else (4, 512, 1024)
    counts = _counts(e, 32) if big else [300, 0, 1, 129]
    x, w, counts = _case(32, e, k, n, counts, extra_rows=77)
    g = torch.Generator(device=DEV)
    g.manual_seed(33)
    scale = torch.rand(e, n, generator=g, device=DEV) * 9e-3 + 1e-3
    pts = torch.rand(x.shape[0], generator=g, device=DEV) * 9e-3 + 1e-3
    out = torch.ops.npu.npu_grouped_matmul([x], [w], scale=[scale], per_token_scale=[pts] if with_pts else None,
                                           group_list=counts, split_item=3, group_type=0, group_list_type=1,
                                           output_dtype=out_dtype)[0]
    acc = _exact(x, w, counts).to(torch.float32)
    row_scale = torch.zeros_like(acc)
    b0 = 0
    for ei, c in enumerate(counts.tolist()):
        row_scale[b0:b0 + c] = scale[ei]
        b0 += c
    want = acc * row_scale
    if with_pts:
        want = want * pts[:, None]
    want = want.to(out_dtype)
    bits = torch.int16 if out_dtype != torch.float32 else torch.int32
    bad = (out.view(bits) != want.view(bits)).nonzero()
    if bad.numel():
        r, c = bad[0].tolist()
        raise AssertionError(f"{bad.shape[0]} of {out.numel()} differ; rows {bad[:, 0].unique()[:8].tolist()}, "
                             f"cols {bad[:, 1].unique()[:8].tolist()}; first [{r},{c}]: got {out[r, c].item()!r} "
                             f"want {want[r, c].item()!r} (fp32 {(acc[r, c] * row_scale[r, c]).item()!r})")


def test_grouped_matches_after_a_different_group_list():
    """Two calls in a row with different group lists (the tile table is rebuilt)."""
    e, k, n = 16, 256, 4096
    for seed in (34, 35):
        x, w, counts = _case(seed, e, k, n, _counts(e, seed), extra_rows=seed - 34)
        out = torch.ops.npu.npu_grouped_matmul([x], [w], group_list=counts, split_item=3, group_type=0,
                                               group_list_type=1, output_dtype=torch.int32)[0]
        assert torch.equal(out.to(torch.int64), _exact(x, w, counts)), f"seed {seed}"
