"""GPU: tai_grouped_matmul_noalloc (scratch in a static device array) against tai_grouped_matmul
(caller workspace), both called through the C ABI, on two calls in a row, the second smaller: the
int32 and bf16 outputs must be identical bit for bit. Also the size limit error."""
import numpy as np
import pytest
import torch

import torchair_amd  # noqa: F401
from oracle import golden as G
from torchair_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _p(t):
    return None if t is None else t.data_ptr()


def _run(entry, x, w, gl, scale, pts, out_dt):
    m, k = x.shape
    e, _, n = w.shape
    out = torch.full((m, n), 7, dtype=out_dt, device=DEV)  # garbage: every element must be written
    code = {torch.int32: _lib.DT_INT32, torch.bfloat16: _lib.DT_BF16}[out_dt]
    stream = torch.cuda.current_stream().cuda_stream
    common = (_p(x), _p(w), m, k, n, e, _lib.LAYOUT_KN, _p(gl), 1, _p(scale), _p(pts), None, _lib.DT_NONE, code,
              _p(out))
    if entry == "ws":
        nb = _lib.query("tai_grouped_matmul_workspace_size", m, n, e)
        ws = torch.empty(nb, dtype=torch.uint8, device=DEV)
        _lib.call("tai_grouped_matmul", *common, _p(ws), nb, stream)
    else:
        _lib.call("tai_grouped_matmul_noalloc", *common, stream)
    return out


@pytest.mark.parametrize("out_dt", [torch.int32, torch.bfloat16])
def test_noalloc_matches_workspace_entry_point(out_dt):
    g = torch.Generator().manual_seed(77)
    # first call: 64 experts with skewed counts, then a smaller call (fewer rows, fewer groups) that
    # reuses the same scratch, whose previous contents must not leak into the result
    for e, m, k, n, hi in ((64, 6000, 512, 512, 64), (8, 700, 256, 256, 3)):
        counts = torch.bincount(torch.randint(0, hi, (m - 9,), generator=g), minlength=e).to(torch.int64)
        x = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8).to(DEV)
        w = torch.randint(-127, 128, (e, k, n), generator=g, dtype=torch.int8).to(DEV)
        sc = (torch.rand(e, n, generator=g) * 9e-3 + 1e-3).to(DEV) if out_dt != torch.int32 else None
        pts = (torch.rand(m, generator=g) * 9e-3 + 1e-3).to(DEV) if out_dt != torch.int32 else None
        gl = counts.to(DEV)
        want = _run("ws", x, w, gl, sc, pts, out_dt)
        got = _run("noalloc", x, w, gl, sc, pts, out_dt)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"e={e} m={m}"
        if out_dt == torch.int32:
            ref = G.grouped_matmul(x.cpu().numpy(), w.cpu().numpy(), counts.numpy(), 1, out_dtype="int32")
            np.testing.assert_array_equal(got.cpu().numpy(), ref)


def test_noalloc_rejects_sizes_beyond_its_scratch():
    limit = _lib.query("tai_grouped_matmul_noalloc_max_scratch")
    m = 1 << 20
    assert _lib.query("tai_grouped_matmul_workspace_size", m, 64, 8) > limit
    # real buffers of the full problem size, so that the call would stay in bounds even if the size
    # check were ever bypassed
    x = torch.zeros(m, 64, dtype=torch.int8, device=DEV)
    w = torch.zeros(8, 64, 64, dtype=torch.int8, device=DEV)
    gl = torch.full((8,), m // 8, dtype=torch.int64, device=DEV)
    out = torch.empty(m, 64, dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match="no-allocation"):
        _lib.call("tai_grouped_matmul_noalloc", x.data_ptr(), w.data_ptr(), m, 64, 64, 8, _lib.LAYOUT_KN,
                  gl.data_ptr(), 1, None, None, None, _lib.DT_NONE, _lib.DT_INT32, out.data_ptr(), None)
    torch.cuda.synchronize()
