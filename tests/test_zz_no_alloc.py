"""hkhip_mm_noalloc, the product that allocates nothing, against the existing entry points it
stands for (hkhip_qact into a caller's buffer, then hkhip_mm), through the C ABI: bit for bit,
on calls in a row whose second input is smaller, so the library's fixed activation buffer is
reused with the first call's contents still in it."""
from __future__ import annotations

import numpy as np
import pytest

from hk_amd import formats as F
from hk_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def setup():
    import torch

    from hk_amd import Engine

    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    e = Engine(0)
    e.set_stream(torch.cuda.current_stream().cuda_stream)
    yield torch, e
    e.close()


def _both(torch, e, w, x, n, bias=None, mode=0, y0=None):
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    bd = None if bias is None else torch.from_numpy(bias).cuda()
    cols = w.rows // 2 if mode == 2 else w.rows
    init = (lambda: torch.from_numpy(y0.copy()).cuda()) if y0 is not None else \
        (lambda: torch.full((n, cols), float("nan"), device="cuda"))
    ya, yb = init(), init()
    xq = torch.empty(e.act_bytes(n, w.cols), dtype=torch.uint8, device="cuda")
    e.qact(xd, n, w.cols, F.ACT_KIND[w.t], xq)
    e.mm(w, xq, ya, n, bd, mode)
    e.mm_noalloc(w, xd, yb, n, bd, mode)
    torch.cuda.synchronize()
    return ya.cpu().numpy(), yb.cpu().numpy()


@pytest.mark.parametrize("t", [F.Q4_K, F.Q6_K, F.Q8_0, F.IQ4_NL, F.Q5_K, F.Q4_1])
@pytest.mark.parametrize("n1,n2", [(512, 1), (40, 8), (12, 3)])
def test_noalloc_matches_mm_twice(setup, t, n1, n2):
    torch, e = setup
    m, k = 700, 2048
    raw = synth.weights_np(t, m, k, seed=3000 + t)
    w = e.upload(raw, t, m, k)
    bias = np.linspace(-1, 1, m).astype(np.float32)
    for i, n in enumerate((n1, n2)):  # the second call smaller: the buffer keeps the first's bytes
        x = synth.activations_np(n, k, seed=3001 + i, outliers=0.01)
        y0 = synth.activations_np(n, m, seed=3003 + i)
        a, b = _both(torch, e, w, x, n, bias=bias, mode=1, y0=y0)
        assert np.isfinite(a).all()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (t, n)
    e.free(w)


def test_noalloc_silu_mul_and_limit(setup):
    from hk_amd import HipError

    torch, e = setup
    t, m, k = F.Q4_K, 2 * 300, 4096
    w = e.upload(synth.weights_np(t, m, k, seed=3010), t, m, k)
    for n in (8, 1):
        a, b = _both(torch, e, w, synth.activations_np(n, k, seed=3011 + n), n, mode=2)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # over the buffer: 2048 tokens at cols 14336 need ~77 MiB; refused before any launch
    big = e.upload(synth.weights_np(t, 16, 14336, seed=3012), t, 16, 14336)
    x = torch.zeros(2048, 14336, device="cuda")
    y = torch.zeros(2048, 16, device="cuda")
    with pytest.raises(HipError) as err:
        e.mm_noalloc(big, x, y, 2048)
    assert err.value.code == -2 and "over its" in str(err.value)
    e.free(w)
    e.free(big)
