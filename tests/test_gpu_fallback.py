"""The float-decode formats (Q2_K, Q3_K, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M,
TQ1_0, TQ2_0, MXFP4, NVFP4) on the GPU, through the C ABI, against the oracle: decoded weights bit
for bit (reference fixtures and random blocks); products against hk's fallback dots
(vecdot.zig:620-720) on the activation form hk pairs with each format (Q8K, A8 for MXFP4, the f32
input for NVFP4), max relative error 1e-3 (tests.helpers.parity_err)."""
from __future__ import annotations

import numpy as np
import pytest

from hk_amd import formats as F
from hk_amd import synth
from hk_amd.engine import ACCUMULATE, SILU_MUL
from oracle import oracle as O
from tests.helpers import PARITY_TOL, load_fixture, parity_err

pytestmark = pytest.mark.gpu

FB = list(F.FALLBACK)


@pytest.fixture(scope="module")
def torch_cuda():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    return torch


@pytest.fixture(scope="module")
def eng(torch_cuda):
    from hk_amd import Engine

    e = Engine(0)
    e.set_stream(torch_cuda.cuda.current_stream().cuda_stream)
    yield e
    e.close()


@pytest.mark.parametrize("t", FB)
def test_fallback_dequant_bit_exact(eng, torch_cuda, t):
    torch = torch_cuda
    fx = load_fixture(F.NAMES[t])
    rows, k = fx["rows"], fx["blocks_per_row"] * fx["block_elems"]
    for raw, r0 in ((fx["raw"], 0), (synth.weights_np(t, 11, 512, seed=4300 + t), 2)):
        rows, k = raw.shape[0], raw.shape[1] // F.INFO[t][1] * F.INFO[t][0]
        w = eng.upload(raw, t, rows, k)
        out = torch.empty((rows - r0, k), dtype=torch.float32, device="cuda")
        eng.dequantize(w, out, row0=r0, nrows=rows - r0)
        got = out.cpu().numpy()
        want = np.stack([O.dequantize(t, raw[r], k) for r in range(r0, rows)])
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        eng.free(w)
    got_fx = np.stack([O.dequantize(t, fx["raw"][r], fx["blocks_per_row"] * fx["block_elems"]) for r in range(fx["rows"])])
    assert np.array_equal(got_fx, fx["expected"])  # gguf's values


@pytest.mark.parametrize("t", FB)
@pytest.mark.parametrize("n", [1, 3, 8, 20])
@pytest.mark.parametrize("prepared", [False, True])
def test_fallback_products(eng, torch_cuda, t, n, prepared):
    """q/k/v-style parts with bias on an f32 input (quantized in the kernel) or a prepared one,
    n up to 8 in one pass; 20 tokens through hkhip_mm (decode passes) with accumulate."""
    torch = torch_cuda
    if prepared and t == F.NVFP4:
        pytest.skip("NVFP4 is dotted against the f32 input (vecdot.zig:189): no prepared form")
    k = 1024
    heights = [70, 33]
    raws = [synth.weights_np(t, m, k, seed=4400 + i + t) for i, m in enumerate(heights)]
    x = synth.activations_np(n, k, seed=4401 + n, outliers=0.01)
    mats = [eng.upload(r, t, m, k) for r, m in zip(raws, heights)]
    xd = torch.from_numpy(x).cuda()
    biases = [torch.from_numpy(np.linspace(-1, 1, m).astype(np.float32)).cuda() for m in heights]
    if n <= 8:
        ys = [torch.full((n, m), float("nan"), device="cuda") for m in heights]
        if prepared:
            xq = torch.empty(eng.act_bytes(n, k), dtype=torch.uint8, device="cuda")
            eng.qact(xd, n, k, F.ACT_KIND[t], xq)
            eng.matvec_parts(mats, ys, n, xq=xq, biases=biases)
        else:
            eng.matvec_parts(mats, ys, n, x=xd, biases=biases)
        y0s = [None, None]
    else:
        y0s = [synth.activations_np(n, m, seed=4402 + m) for m in heights]
        ys = [torch.from_numpy(y0.copy()).cuda() for y0 in y0s]
        for w, y, b in zip(mats, ys, biases):
            if prepared:
                xq = torch.empty(eng.act_bytes(n, k), dtype=torch.uint8, device="cuda")
                eng.qact(xd, n, k, F.ACT_KIND[t], xq)
                eng.mm(w, xq, y, n, bias=b, mode=ACCUMULATE)
            else:
                eng.mm_noalloc(w, xd, y, n, bias=b, mode=ACCUMULATE)
    torch.cuda.synchronize()
    for r, m, y, b, y0 in zip(raws, heights, ys, biases, y0s):
        want = O.matmul(t, r, m, k, x, n, bias=b.cpu().numpy())
        if y0 is not None:
            want = want + y0
        assert parity_err(y.cpu().numpy(), want) <= PARITY_TOL
    for w in mats:
        eng.free(w)


@pytest.mark.parametrize("t", [F.Q2_K, F.IQ2_XS, F.MXFP4, F.NVFP4])
def test_fallback_silu_mul_and_host_gemv(eng, torch_cuda, t):
    from hk_amd import gemm

    torch = torch_cuda
    k, m, n = 512, 2 * 40, 3
    raw = synth.weights_np(t, m, k, seed=4500 + t)
    x = synth.activations_np(n, k, seed=4501)
    w = eng.upload(raw, t, m, k)
    y = torch.full((n, m // 2), float("nan"), device="cuda")
    eng.matvec_parts([w], [y], n, x=torch.from_numpy(x).cuda(), mode=SILU_MUL)
    torch.cuda.synchronize()
    ref = O.matmul(t, raw, m, k, x, n).astype(np.float32)
    g, u = ref[:, 0::2], ref[:, 1::2]
    with np.errstate(over="ignore"):
        want = g / (np.float32(1) + np.exp(-g)) * u
    assert parity_err(y.cpu().numpy(), want) <= PARITY_TOL
    eng.free(w)
    bias = np.arange(m, dtype=np.float32)
    got = gemm(t, raw, x, bias, m, k, n)  # host pointers (hk_gemv-style entry point)
    assert parity_err(got, O.matmul(t, raw, m, k, x, n, bias=bias)) <= PARITY_TOL


def test_fallback_rejects(eng, torch_cuda):
    from hk_amd import HipError

    torch = torch_cuda
    w = eng.upload(synth.weights_np(F.NVFP4, 4, 256, seed=1), F.NVFP4, 4, 256)
    xq = torch.zeros(eng.act_bytes(1, 256), dtype=torch.uint8, device="cuda")
    with pytest.raises(HipError) as e:
        eng.matvec(w, xq, torch.zeros(1, 4, device="cuda"), 1)  # NVFP4 needs the f32 input
    assert e.value.code == -1
    eng.free(w)
    w = eng.upload(synth.weights_np(F.MXFP4, 4, 96, seed=2), F.MXFP4, 4, 96)  # uploads; products need 256-multiples
    with pytest.raises(HipError) as e:
        eng.matvec_parts([w], [torch.zeros(1, 4, device="cuda")], 1, x=torch.zeros(1, 96, device="cuda"))
    assert e.value.code == -2
    eng.free(w)
