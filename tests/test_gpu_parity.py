"""GPU parity: the HIP kernels, called through the C ABI, against the CPU oracle.

Bars: dequantized weights and quantized activations bit-identical to hk's CPU arithmetic;
matvec / GEMM outputs within max relative error 1e-3 (helpers.parity_err) of the oracle's
restatement of hk's CPU kernels on the same seeded inputs. Shapes follow the reference's own
GPU parity tests (tests/test_cuda.zig:287-389: M = 21, K = 512, n in {1, 19, 150}) plus ragged
rows, the smallest legal K, bias, accumulate mode and the BASELINE shapes.
"""
from __future__ import annotations

import numpy as np
import pytest

from hk_amd import formats as F
from hk_amd import synth
from hk_amd.engine import ACCUMULATE, SILU_MUL
from oracle import oracle as O
from tests.helpers import PARITY_TOL, load_fixture, parity_err, tie_rows

pytestmark = pytest.mark.gpu

FMTS = [F.Q8_0, F.Q4_K, F.Q6_K, F.IQ4_NL, F.Q4_0, F.Q4_1, F.Q5_0, F.Q5_1, F.Q5_K, F.IQ4_XS]
FIXTURES = F.NAMES
LOW4 = [F.Q4_0, F.Q4_1, F.Q5_0, F.Q5_1]


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


def run(eng, torch, t, raw, m, k, x, path="mm", bias=None, mode=0, y0=None):
    n = x.shape[0]
    w = eng.upload(raw, t, m, k)
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    xq = torch.empty(eng.act_bytes(n, k), dtype=torch.uint8, device="cuda")
    eng.qact(xd, n, k, F.ACT_KIND[t], xq)
    y = torch.from_numpy(y0.copy()).cuda() if y0 is not None else torch.full((n, m), float("nan"), device="cuda")
    bd = torch.from_numpy(bias).cuda() if bias is not None else None
    getattr(eng, path)(w, xq, y, n, bd, mode)
    torch.cuda.synchronize()
    out = y.cpu().numpy()
    eng.free(w)
    return out


# ---------------------------------------------------------------------------------------- dequant

@pytest.mark.parametrize("t", FMTS)
def test_dequant_fixture_bit_exact(eng, torch_cuda, t):
    fx = load_fixture(FIXTURES[t])
    rows, k = fx["rows"], fx["blocks_per_row"] * fx["block_elems"]
    w = eng.upload(fx["raw"], t, rows, k)
    out = torch_cuda.empty((rows, k), dtype=torch_cuda.float32, device="cuda")
    eng.dequantize(w, out)
    got = out.cpu().numpy()
    want = np.stack([O.dequantize(t, fx["raw"][r], k) for r in range(rows)])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(got, fx["expected"])  # gguf's values (equal up to the sign of zero)
    eng.free(w)


@pytest.mark.parametrize("t", FMTS)
def test_dequant_random_bit_exact(eng, torch_cuda, t):
    rows, k = 13, 1024
    raw = synth.weights_np(t, rows, k, seed=7 + t)
    w = eng.upload(raw, t, rows, k)
    out = torch_cuda.empty((rows - 3, k), dtype=torch_cuda.float32, device="cuda")
    eng.dequantize(w, out, row0=3, nrows=rows - 3)
    got = out.cpu().numpy()
    want = np.stack([O.dequantize(t, raw[r], k) for r in range(3, rows)])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    eng.free(w)


# ---------------------------------------------------------------------------------------- qact

def _act_cases():
    rng = np.random.default_rng(11)
    x = rng.normal(0, 1, (5, 1024)).astype(np.float32)
    x[1, :256] = 0.0                      # an all-zero super-block and eight zero A8 blocks
    x[2, 3] = 7.5
    x[2, 200] = -7.5                      # tie on |x|: the first one sets the sign of d
    x[3] *= 1e-30                         # tiny (denormal-range) values
    x[4] = synth.activations_np(1, 1024, 3, outliers=0.01)[0]
    return np.concatenate([x, tie_rows(1024)[0]])  # ties k + 0.5 at scale 1: round half away


@pytest.mark.parametrize("kind", [F.ACT_A8, F.ACT_Q8K])
def test_qact_bit_exact(eng, torch_cuda, kind):
    x = _act_cases()
    n, k = x.shape
    xd = torch_cuda.from_numpy(x).cuda()
    xq = torch_cuda.empty(eng.act_bytes(n, k), dtype=torch_cuda.uint8, device="cuda")
    eng.qact(xd, n, k, kind, xq)
    got = eng.act_export(xq, n, k, kind)
    want = np.concatenate([(O.quantize_a8 if kind == F.ACT_A8 else O.quantize_q8k)(x[i]) for i in range(n)])
    assert np.array_equal(got, want.view(np.uint8))
    tie = want[-(k // (32 if kind == F.ACT_A8 else 256)):]
    assert np.array_equal(tie["qs"].astype(np.int64).ravel(), tie_rows(k)[1][0])  # the closed form


@pytest.mark.parametrize("t", FMTS)
def test_in_kernel_qact_rounds_ties_away(eng, torch_cuda, t):
    """The decode kernels' own quantization of an f32 input, on tie values (tests.helpers.tie_rows):
    rounding them to even instead of away from zero moves the outputs by several percent."""
    torch = torch_cuda
    m, k = 200, 1024
    raw = synth.weights_np(t, m, k, seed=2100 + t)
    x = tie_rows(k)[0]
    w = eng.upload(raw, t, m, k)
    y = torch.full((1, m), float("nan"), device="cuda")
    eng.matvec_parts([w], [y], 1, x=torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    assert parity_err(y.cpu().numpy(), O.matmul(t, raw, m, k, x, 1, tiled=False)) <= PARITY_TOL
    eng.free(w)


# ---------------------------------------------------------------------------------------- products

MATVEC_SHAPES = [(21, 512), (300, 1024), (64, 256), (1, 4096), (37, 3072)]


@pytest.mark.parametrize("t", FMTS)
@pytest.mark.parametrize("n", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("shape", MATVEC_SHAPES)
def test_matvec_parity(eng, torch_cuda, t, n, shape):
    m, k = shape
    raw = synth.weights_np(t, m, k, seed=100 + m + t)
    x = synth.activations_np(n, k, seed=200 + n)
    got = run(eng, torch_cuda, t, raw, m, k, x, path="matvec")
    want = O.matmul(t, raw, m, k, x, n, tiled=False)
    assert parity_err(got, want) <= PARITY_TOL


GEMM_SHAPES = [(21, 512), (37, 256), (130, 1024), (64, 3072)]


@pytest.mark.parametrize("t", FMTS)
@pytest.mark.parametrize("n", [1, 8, 11, 19, 150])
@pytest.mark.parametrize("shape", GEMM_SHAPES)
def test_gemm_parity(eng, torch_cuda, t, n, shape):
    m, k = shape
    raw = synth.weights_np(t, m, k, seed=300 + m + t)
    x = synth.activations_np(n, k, seed=400 + n, outliers=0.01)
    got = run(eng, torch_cuda, t, raw, m, k, x, path="gemm")
    want = O.matmul(t, raw, m, k, x, n, tiled=True)
    assert parity_err(got, want) <= PARITY_TOL


@pytest.mark.parametrize("t", FMTS)
def test_fixture_rows_gemm(eng, torch_cuda, t):
    """The reference's tiled-GEMM test shape (test_quant.zig:281-359): 37 rows tiled from the
    fixture rows, 11 tokens, bias i % 5."""
    fx = load_fixture(FIXTURES[t])
    k = fx["blocks_per_row"] * fx["block_elems"]
    raw = np.stack([fx["raw"][r % fx["rows"]] for r in range(37)])
    x = np.random.default_rng(0x6E33).uniform(-1, 1, (11, k)).astype(np.float32)
    bias = (np.arange(37) % 5).astype(np.float32)
    got = run(eng, torch_cuda, t, raw, 37, k, x, path="mm", bias=bias)
    want = O.matmul(t, raw, 37, k, x, 11, bias=bias)
    assert parity_err(got, want) <= PARITY_TOL


@pytest.mark.parametrize("t", FMTS)
@pytest.mark.parametrize("n", [7, 8])
def test_mm_dispatch_bias_accumulate(eng, torch_cuda, t, n):
    m, k = 45, 512
    raw = synth.weights_np(t, m, k, seed=500 + t)
    x = synth.activations_np(n, k, seed=501)
    bias = np.linspace(-2, 2, m).astype(np.float32)
    y0 = synth.activations_np(n, m, seed=502)
    got = run(eng, torch_cuda, t, raw, m, k, x, path="mm", bias=bias, mode=1, y0=y0)
    want = O.matmul(t, raw, m, k, x, n, bias=bias) + y0
    assert parity_err(got, want) <= PARITY_TOL



@pytest.mark.parametrize("t", FMTS)
@pytest.mark.parametrize("n", [9, 17, 24, 40])
def test_mm_chunked_matvec(eng, torch_cuda, t, n):
    """hkhip_mm between 8 tokens and the GEMM's break-even runs 8-token matvec passes (a ragged
    last one); bias and accumulate apply once per token."""
    m, k = 300, 1024
    raw = synth.weights_np(t, m, k, seed=700 + t)
    x = synth.activations_np(n, k, seed=701 + n)
    bias = np.linspace(-1, 1, m).astype(np.float32)
    y0 = synth.activations_np(n, m, seed=702)
    got = run(eng, torch_cuda, t, raw, m, k, x, path="mm", bias=bias, mode=1, y0=y0)
    want = O.matmul(t, raw, m, k, x, n, bias=bias) + y0
    assert parity_err(got, want) <= PARITY_TOL

@pytest.mark.parametrize("t", LOW4)
@pytest.mark.parametrize("n", [9, 30, 40])
def test_low4_rows_not_whole_super_blocks(eng, torch_cuda, t, n):
    """Q4_0..Q5_1 with K = 96 (three blocks, no whole super-block): the GEMM entry points run
    decode passes; bias and accumulate."""
    m, k = 45, 96
    raw = synth.weights_np(t, m, k, seed=1500 + t)
    x = synth.activations_np(n, k, seed=1501)
    bias = np.arange(m, dtype=np.float32)
    y0 = synth.activations_np(n, m, seed=1502)
    for path in ("mm", "gemm"):
        got = run(eng, torch_cuda, t, raw, m, k, x, path=path, bias=bias, mode=1, y0=y0)
        want = O.matmul(t, raw, m, k, x, n, bias=bias) + y0
        assert parity_err(got, want) <= PARITY_TOL


def test_host_gemv_q4_0_symbol(torch_cuda):
    """hkhip_gemv_q4_0 stands in for hk_gemv_q4_0 (hk.h:452): host pointers, bias."""
    import ctypes
    from hk_amd import _lib

    m, k = 19, 512
    raw = np.ascontiguousarray(synth.weights_np(F.Q4_0, m, k, seed=1600))
    x = synth.activations_np(1, k, seed=1601)[0]
    bias = np.linspace(-2, 2, m).astype(np.float32)
    y = np.full(m, np.nan, np.float32)
    P = ctypes.c_void_p
    rc = _lib.lib().hkhip_gemv_q4_0(raw.ctypes.data_as(P), x.ctypes.data_as(P), bias.ctypes.data_as(P),
                                    y.ctypes.data_as(P), m, k)
    assert rc == 0
    want = O.matmul(F.Q4_0, raw, m, k, x[None], 1, bias=bias)[0]
    assert parity_err(y, want) <= PARITY_TOL


def test_host_gemv_entry_points(torch_cuda):
    from hk_amd import gemm, gemv

    m, k = 33, 1024
    for t in FMTS:
        raw = synth.weights_np(t, m, k, seed=600 + t)
        x = synth.activations_np(1, k, seed=601)
        bias = np.arange(m, dtype=np.float32)
        got = gemv(t, raw, x[0], bias, m, k)
        want = O.matmul(t, raw, m, k, x, 1, bias=bias)[0]
        assert parity_err(got, want) <= PARITY_TOL
        xs = synth.activations_np(12, k, seed=602)
        got = gemm(t, raw, xs, None, m, k, 12)
        assert parity_err(got, O.matmul(t, raw, m, k, xs, 12)) <= PARITY_TOL


def test_errors(eng, torch_cuda):
    from hk_amd import HipError
    from hk_amd import gemm as host_gemm

    with pytest.raises(HipError) as e:
        eng.upload(np.zeros(100 * 34 // 32, np.uint8), F.Q8_0, 1, 100)
    assert e.value.code == -2  # UNSUPPORTED_SHAPE: cols not a multiple of 32
    with pytest.raises(HipError) as e:
        eng.upload(np.zeros(512, np.uint8), 0x01, 1, 256)  # f16: not on this path
    assert e.value.code == -1
    raw = synth.weights_np(F.Q4_K, 4, 256, seed=1)
    w = eng.upload(raw, F.Q4_K, 4, 256)
    xq = torch_cuda.zeros(eng.act_bytes(9, 256), dtype=torch_cuda.uint8, device="cuda")
    y = torch_cuda.zeros((9, 4), device="cuda")
    with pytest.raises(HipError):
        eng.matvec(w, xq, y, 9)  # decode kernels take at most 8 tokens
    with pytest.raises(HipError):
        eng.mm(w, xq, y, 2, None, 7)  # unknown mode
    eng.free(w)
    with pytest.raises(HipError) as e:
        host_gemm(F.Q4_K, np.zeros(144, np.uint8), np.zeros(100, np.float32), None, 1, 100, 1)
    assert np.isnan(e.value.y).all()  # hk's C ABI poisons the output (c_api.zig:16-18)


# ---------------------------------------------------------------------------------------- BASELINE shapes

@pytest.mark.parametrize("t,m,k,n", [
    (F.Q8_0, 3072, 1024, 1),        # config 1
    (F.Q4_K, 14336, 4096, 1),       # config 4 gate/up
    (F.Q4_K, 4096, 14336, 8),       # config 4 down, batch 8
    (F.IQ4_NL, 14336, 4096, 1),     # config 5
    (F.Q6_K, 4096, 14336, 1),       # config 5 down
])
def test_baseline_matvec_shapes(eng, torch_cuda, t, m, k, n):
    raw = synth.weights_np(t, m, k, seed=synth.seed_for(4, t))
    x = synth.activations_np(n, k, seed=synth.seed_for(4, 99), outliers=0.01 if t == F.IQ4_NL else 0.0)
    got = run(eng, torch_cuda, t, raw, m, k, x, path="mm")
    want = O.matmul(t, raw, m, k, x, n, threads=16)
    assert parity_err(got, want) <= PARITY_TOL


@pytest.mark.parametrize("t,m,k", [(F.Q4_K, 3072, 1024), (F.Q4_K, 1024, 3072), (F.Q6_K, 1024, 3072),
                                   (F.IQ4_NL, 3072, 1024)])
def test_baseline_prefill_shapes(eng, torch_cuda, t, m, k):
    n = 512  # config 3
    raw = synth.weights_np(t, m, k, seed=synth.seed_for(3, t))
    x = synth.activations_np(n, k, seed=synth.seed_for(3, 99))
    got = run(eng, torch_cuda, t, raw, m, k, x, path="mm")
    want = O.matmul(t, raw, m, k, x, n, threads=16)
    assert parity_err(got, want) <= PARITY_TOL


@pytest.mark.parametrize("t,m,k,n,mode", [(F.IQ4_NL, 4000, 1280, 300, 1), (F.IQ4_NL, 9000, 512, 260, 0),
                                          (F.Q6_K, 4100, 768, 100, 1), (F.Q8_0, 3000, 1024, 70, 1)] +
                         [(t, 4000, 1280, 300, 1) for t in LOW4 + [F.IQ4_XS]] +
                         [(t, 9000, 512, 260, 0) for t in LOW4 + [F.IQ4_XS]] + [(F.IQ4_XS, 1000, 768, 50, 0),
                                                                        (F.Q5_K, 4000, 1280, 300, 1), (F.Q5_K, 9000, 512, 260, 0),
                                                                        (F.Q5_K, 1000, 768, 50, 1),
                                                                        (F.Q5_K, 12288, 512, 520, 1), (F.Q5_K, 12300, 768, 512, 0),
                                                                        (F.Q5_K, 4096, 1024, 512, 1), (F.Q5_K, 4100, 768, 330, 0)] +
                         # 64-row tiles over K slices: few row blocks (K 4096), or few tokens
                         [(t, 1000, 4096, 40, 1) for t in (F.Q4_1, F.Q5_0, F.Q5_1, F.IQ4_XS)] +
                         [(t, 9000, 4352, 20, 0) for t in (F.Q4_1, F.Q5_0, F.Q5_1, F.IQ4_XS)])
def test_gemm_configs_other_formats(eng, torch_cuda, t, m, k, n, mode):
    """The configurations of the mmx / mm2 GEMM tiles for the formats other than Q4_K: IQ4_NL over
    two K slices (5 super-blocks) and its 256-row tile; Q6_K and Q8_0 tiles; Q4_0..Q5_1 and IQ4_XS
    on the 256-row tile (9000 rows) and the 128-row two-slice tile (4000 rows, with an uneven
    17-block split at K 1280); the 64-row tiles over K slices (two for Q5_0 / Q5_1, four for Q4_1 /
    IQ4_XS) at cols >= 4096 with few row blocks or few tokens; Q5_K on the Q4_K register tile
    (12288 / 12300 rows) and on mmx / the 128-row ring tile otherwise; ragged rows and tokens,
    bias, accumulate."""
    raw = synth.weights_np(t, m, k, seed=1400 + m)
    x = synth.activations_np(n, k, seed=1401, outliers=0.01)
    bias = np.linspace(-1, 1, m).astype(np.float32) if mode else None
    y0 = synth.activations_np(n, m, seed=1402) if mode else None
    got = run(eng, torch_cuda, t, raw, m, k, x, path="gemm", bias=bias, mode=mode, y0=y0)
    want = O.matmul(t, raw, m, k, x, n, bias=bias, threads=16)
    if mode:
        want = want + y0
    assert parity_err(got, want) <= PARITY_TOL


@pytest.mark.parametrize("m,k,n,mode", [(12288, 256, 512, 0), (12000, 512, 520, 1),
                                        (2000, 2304, 130, 1), (2048, 512, 128, 0), (2600, 1280, 520, 1)])
def test_gemm_large_tile(eng, torch_cuda, m, k, n, mode):
    """Shapes that select each Q4_K GEMM configuration: the 256-row x 128-token register tile (at
    least 192 tiles), and the ring kernel split over 4 and 2 K slices (9 and 5 super-blocks, so
    slices get unequal counts; 2 super-blocks over 2 slices); exact fits and ragged rows and
    tokens with bias and accumulate."""
    t = F.Q4_K
    raw = synth.weights_np(t, m, k, seed=600 + m)
    x = synth.activations_np(n, k, seed=601, outliers=0.01)
    bias = np.linspace(-1, 1, m).astype(np.float32) if mode else None
    y0 = synth.activations_np(n, m, seed=602) if mode else None
    got = run(eng, torch_cuda, t, raw, m, k, x, path="mm", bias=bias, mode=mode, y0=y0)
    want = O.matmul(t, raw, m, k, x, n, bias=bias, threads=16)
    if mode:
        want = want + y0
    assert parity_err(got, want) <= PARITY_TOL


# ---------------------------------------------------------------------------------------- fused parts

@pytest.mark.parametrize("t", FMTS)
@pytest.mark.parametrize("n", [1, 3, 8])
@pytest.mark.parametrize("prepared", [False, True])
def test_matvec_parts_parity(eng, torch_cuda, t, n, prepared):
    """q/k/v-style fusion: three matrices of different heights sharing one input, in one launch,
    with the input quantized inside the kernel (or prepared by qact). Each part is checked
    against the oracle on its own."""
    torch = torch_cuda
    k = 1024
    heights = [96, 32, 40]
    raws = [synth.weights_np(t, m, k, seed=700 + i + t) for i, m in enumerate(heights)]
    x = synth.activations_np(n, k, seed=701 + n, outliers=0.01)
    mats = [eng.upload(r, t, m, k) for r, m in zip(raws, heights)]
    ys = [torch.full((n, m), float("nan"), device="cuda") for m in heights]
    biases = [torch.from_numpy(np.arange(m, dtype=np.float32) * 0.5).cuda() for m in heights]
    xd = torch.from_numpy(x).cuda()
    if prepared:
        xq = torch.empty(eng.act_bytes(n, k), dtype=torch.uint8, device="cuda")
        eng.qact(xd, n, k, F.ACT_KIND[t], xq)
        eng.matvec_parts(mats, ys, n, xq=xq, biases=biases)
    else:
        eng.matvec_parts(mats, ys, n, x=xd, biases=biases)
    torch.cuda.synchronize()
    for r, m, y, b in zip(raws, heights, ys, biases):
        want = O.matmul(t, r, m, k, x, n, bias=b.cpu().numpy(), tiled=False)
        assert parity_err(y.cpu().numpy(), want) <= PARITY_TOL
    for w in mats:
        eng.free(w)


@pytest.mark.parametrize("t,k,n", [(F.Q4_K, 14336, 8), (F.Q8_0, 20480, 8), (F.Q6_K, 4096, 8)])
def test_matvec_parts_large_k(eng, torch_cuda, t, k, n):
    """The largest decode inputs: 8 tokens of the 8B down projection (~130 KB of activations in
    LDS) and, for Q8_0, more than the LDS holds (the launch splits the tokens)."""
    torch = torch_cuda
    m = 300
    raw = synth.weights_np(t, m, k, seed=800 + t)
    x = synth.activations_np(n, k, seed=801)
    w = eng.upload(raw, t, m, k)
    y = torch.full((n, m), float("nan"), device="cuda")
    eng.matvec_parts([w], [y], n, x=torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    assert parity_err(y.cpu().numpy(), O.matmul(t, raw, m, k, x, n, tiled=False)) <= PARITY_TOL
    eng.free(w)


# ---------------------------------------------------------------------------------------- kernel variants

@pytest.mark.parametrize("t,k,n", [
    (F.Q4_K, 4096, 1), (F.Q4_K, 8192, 1), (F.Q4_K, 16384, 1), (F.Q4_K, 16640, 1),   # C=1,2,4, LDS kernel
    (F.Q4_K, 8192, 2), (F.Q4_K, 16384, 2), (F.Q4_K, 8192, 4), (F.Q4_K, 4096, 5), (F.Q4_K, 8192, 8),
    (F.Q6_K, 8192, 1), (F.Q6_K, 16384, 1), (F.Q6_K, 8192, 2), (F.Q6_K, 4096, 4), (F.Q6_K, 4096, 7),
    (F.Q8_0, 2048, 1), (F.Q8_0, 16384, 1), (F.Q8_0, 16416, 1), (F.Q8_0, 8192, 2), (F.Q8_0, 4096, 6),
    (F.IQ4_NL, 8192, 1), (F.IQ4_NL, 16384, 2), (F.IQ4_NL, 4096, 8), (F.IQ4_NL, 96, 3),
    # rows split over 2-8 waves (K slices), partials combined in LDS
    (F.Q4_K, 14336, 8), (F.Q4_K, 14336, 2), (F.Q4_K, 14336, 3), (F.Q4_K, 28672, 1),
    (F.Q6_K, 14336, 8), (F.Q6_K, 20480, 1), (F.Q8_0, 20480, 8), (F.IQ4_NL, 14336, 4),
    # the 4/5-bit formats: register kernel C = 8, LDS kernel, K slices
    (F.Q4_0, 16384, 1), (F.Q4_1, 16416, 1), (F.Q5_0, 8192, 2), (F.Q5_1, 4096, 8),
    (F.Q4_0, 14336, 4), (F.Q4_1, 14336, 8), (F.Q5_0, 20480, 1), (F.Q5_1, 16384, 2),
    # Q5_K and IQ4_XS: register kernel, LDS kernel (including the NT = 6-8 variants), K slices
    (F.Q5_K, 8192, 1), (F.Q5_K, 16384, 1), (F.Q5_K, 4096, 2), (F.Q5_K, 4096, 7), (F.Q5_K, 14336, 8),
    (F.IQ4_XS, 16384, 1), (F.IQ4_XS, 8192, 2), (F.IQ4_XS, 4096, 5), (F.IQ4_XS, 14336, 8), (F.IQ4_XS, 16640, 1),
])
@pytest.mark.parametrize("prepared", [False, True])
def test_matvec_kernel_variants(eng, torch_cuda, t, k, n, prepared):
    """Every register-kernel variant (units per lane 1-8, token counts padded up to 1/2/4/8, rows
    split over 2-8 waves) and the shapes past it; f32 input and prepared input."""
    torch = torch_cuda
    m = 333
    raw = synth.weights_np(t, m, k, seed=900 + t + k)
    x = synth.activations_np(n, k, seed=901 + n, outliers=0.01)
    w = eng.upload(raw, t, m, k)
    y = torch.full((n, m), float("nan"), device="cuda")
    xd = torch.from_numpy(x).cuda()
    if prepared:
        xq = torch.empty(eng.act_bytes(n, k), dtype=torch.uint8, device="cuda")
        eng.qact(xd, n, k, F.ACT_KIND[t], xq)
        eng.matvec_parts([w], [y], n, xq=xq)
    else:
        eng.matvec_parts([w], [y], n, x=xd)
    torch.cuda.synchronize()
    assert parity_err(y.cpu().numpy(), O.matmul(t, raw, m, k, x, n, tiled=False)) <= PARITY_TOL
    eng.free(w)


def test_matvec_many_rows_per_wave(eng, torch_cuda):
    """More rows than a wave keeps results for (64), so results are stored in several batches;
    accumulate mode and a bias on top."""
    torch = torch_cuda
    t, m, k, n = F.Q8_0, 140000, 256, 2
    raw = synth.weights_np(t, m, k, seed=950)
    x = synth.activations_np(n, k, seed=951)
    w = eng.upload(raw, t, m, k)
    y0 = np.random.default_rng(952).standard_normal((n, m)).astype(np.float32)
    y = torch.from_numpy(y0).cuda()
    b = torch.from_numpy(np.linspace(-1, 1, m, dtype=np.float32)).cuda()
    eng.matvec_parts([w], [y], n, x=torch.from_numpy(x).cuda(), biases=[b], mode=ACCUMULATE)
    torch.cuda.synchronize()
    want = y0 + O.matmul(t, raw, m, k, x, n, bias=b.cpu().numpy(), tiled=False)
    assert parity_err(y.cpu().numpy(), want) <= PARITY_TOL
    eng.free(w)


@pytest.mark.parametrize("t", FMTS)
def test_matvec_parts_straddling_waves(eng, torch_cuda, t):
    """Parts large enough that some waves' row ranges cross from one part into the next."""
    torch = torch_cuda
    k, n = 512, 1
    heights = [3001, 999, 1203, 77]
    raws = [synth.weights_np(t, m, k, seed=960 + i) for i, m in enumerate(heights)]
    x = synth.activations_np(n, k, seed=965)
    mats = [eng.upload(r, t, m, k) for r, m in zip(raws, heights)]
    ys = [torch.full((n, m), float("nan"), device="cuda") for m in heights]
    eng.matvec_parts(mats, ys, n, x=torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    for r, m, y in zip(raws, heights, ys):
        assert parity_err(y.cpu().numpy(), O.matmul(t, r, m, k, x, n, tiled=False)) <= PARITY_TOL
    for w in mats:
        eng.free(w)


# ---------------------------------------------------------------------------------------- silu(gate) * up

def silu_mul_ref(y):
    """shaders/mmvq.comp:186 on the oracle's product of interleaved gate/up rows."""
    g, u = y[:, 0::2].astype(np.float32), y[:, 1::2].astype(np.float32)
    with np.errstate(over="ignore"):  # exp(-g) = inf for very negative g: silu -> -0, as on the GPU
        return g / (np.float32(1) + np.exp(-g)) * u


@pytest.mark.parametrize("t", FMTS)
@pytest.mark.parametrize("n", [1, 3, 5, 8])
@pytest.mark.parametrize("prepared", [False, True])
def test_silu_mul_parts(eng, torch_cuda, t, n, prepared):
    """Mode 2 (the Vulkan mmvq's fused gate/up): two interleaved gate/up matrices in one launch,
    each output silu(gate) * up; f32 input (decode kernel) or prepared (Q4_K from 4 tokens: the
    small-batch kernel)."""
    torch = torch_cuda
    k = 1024
    heights = [2 * 48, 2 * 21]
    raws = [synth.weights_np(t, m, k, seed=1100 + i + t) for i, m in enumerate(heights)]
    x = synth.activations_np(n, k, seed=1101 + n, outliers=0.01)
    mats = [eng.upload(r, t, m, k) for r, m in zip(raws, heights)]
    ys = [torch.full((n, m // 2), float("nan"), device="cuda") for m in heights]
    xd = torch.from_numpy(x).cuda()
    if prepared:
        xq = torch.empty(eng.act_bytes(n, k), dtype=torch.uint8, device="cuda")
        eng.qact(xd, n, k, F.ACT_KIND[t], xq)
        eng.matvec_parts(mats, ys, n, xq=xq, mode=SILU_MUL)
    else:
        eng.matvec_parts(mats, ys, n, x=xd, mode=SILU_MUL)
    torch.cuda.synchronize()
    for r, m, y in zip(raws, heights, ys):
        want = silu_mul_ref(O.matmul(t, r, m, k, x, n, tiled=False))
        assert parity_err(y.cpu().numpy(), want) <= PARITY_TOL
    for w in mats:
        eng.free(w)


@pytest.mark.parametrize("t,k,n", [(F.Q4_K, 14336, 8), (F.Q4_K, 16640, 1), (F.Q8_0, 16416, 2),
                                   (F.Q6_K, 20480, 1), (F.IQ4_NL, 4096, 8), (F.Q4_K, 4096, 1),
                                   (F.Q8_0, 4096, 1), (F.Q4_K, 2048, 1)])
def test_silu_mul_kernel_variants(eng, torch_cuda, t, k, n):
    """Mode 2 where rows are split over K-slice waves, where the LDS kernel runs (rows longer
    than the register kernel takes), and in the one-token register kernels whose steps hold one
    row (rows then stay in contiguous ranges per wave, so a gate/up pair is never split)."""
    torch = torch_cuda
    m = 2 * 150
    raw = synth.weights_np(t, m, k, seed=1200 + t + k)
    x = synth.activations_np(n, k, seed=1201 + n)
    w = eng.upload(raw, t, m, k)
    y = torch.full((n, m // 2), float("nan"), device="cuda")
    eng.matvec_parts([w], [y], n, x=torch.from_numpy(x).cuda(), mode=SILU_MUL)
    torch.cuda.synchronize()
    want = silu_mul_ref(O.matmul(t, raw, m, k, x, n, tiled=False))
    assert parity_err(y.cpu().numpy(), want) <= PARITY_TOL
    eng.free(w)


@pytest.mark.parametrize("t", FMTS)
@pytest.mark.parametrize("n,m", [(9, 2 * 150), (40, 2 * 256), (200, 2 * 150), (64, 2 * 1024)])
def test_silu_mul_gemm(eng, torch_cuda, t, n, m):
    """Mode 2 through hkhip_mm past 8 tokens: the small-batch kernel, the decode passes and the
    GEMMs' epilogues (their LDS-transposed 16-byte stores where rows are a multiple of 8, lane
    pairs otherwise), against the oracle's product of the interleaved rows."""
    torch = torch_cuda
    k = 1024
    raw = synth.weights_np(t, m, k, seed=1250 + t + m)
    x = synth.activations_np(n, k, seed=1251 + n, outliers=0.01)
    w = eng.upload(raw, t, m, k)
    xd = torch.from_numpy(x).cuda()
    xq = torch.empty(eng.act_bytes(n, k), dtype=torch.uint8, device="cuda")
    eng.qact(xd, n, k, F.ACT_KIND[t], xq)
    y = torch.full((n, m // 2), float("nan"), device="cuda")
    eng.mm(w, xq, y, n, mode=SILU_MUL)
    torch.cuda.synchronize()
    want = silu_mul_ref(O.matmul(t, raw, m, k, x, n, tiled=True))
    assert parity_err(y.cpu().numpy(), want) <= PARITY_TOL
    eng.free(w)


def test_silu_mul_gemm_large_tile(eng, torch_cuda):
    """Mode 2 in the Q4_K register-tile GEMM (14336 x 256 at 512 tokens, the prefill gate/up
    shape's tile): the epilogue's output equals silu(gate) * up of the same GEMM's stored rows
    (expf aside, to 1e-6), and sampled gate/up pairs match the oracle."""
    torch = torch_cuda
    t, m, k, n = F.Q4_K, 14336, 256, 512
    raw = synth.weights_np(t, m, k, seed=1260)
    x = synth.activations_np(n, k, seed=1261)
    w = eng.upload(raw, t, m, k)
    xq = torch.empty(eng.act_bytes(n, k), dtype=torch.uint8, device="cuda")
    eng.qact(torch.from_numpy(x).cuda(), n, k, F.ACT_KIND[t], xq)
    y2 = torch.full((n, m), float("nan"), device="cuda")
    ys = torch.full((n, m // 2), float("nan"), device="cuda")
    eng.gemm(w, xq, y2, n)
    eng.gemm(w, xq, ys, n, mode=SILU_MUL)
    torch.cuda.synchronize()
    got = ys.cpu().numpy()
    assert parity_err(got, silu_mul_ref(y2.cpu().numpy())) <= 1e-6
    pairs = np.random.default_rng(1262).choice(m // 2, 24, replace=False)
    rows = np.stack([2 * pairs, 2 * pairs + 1], 1).reshape(-1)
    want = silu_mul_ref(O.matmul(t, raw[rows], len(rows), k, x, n, tiled=True))
    assert parity_err(got[:, pairs], want) <= PARITY_TOL
    eng.free(w)


def test_silu_mul_rejects(eng, torch_cuda):
    """Mode 2 takes an even row count and no bias."""
    from hk_amd import HipError

    torch = torch_cuda
    t, k = F.Q4_K, 256
    odd = eng.upload(synth.weights_np(t, 7, k, seed=1300), t, 7, k)
    even = eng.upload(synth.weights_np(t, 8, k, seed=1301), t, 8, k)
    xq = torch.zeros(eng.act_bytes(16, k), dtype=torch.uint8, device="cuda")
    y = torch.zeros(16, 8, device="cuda")
    b = torch.zeros(8, device="cuda")
    with pytest.raises(HipError):
        eng.matvec(odd, xq, y, 1, mode=SILU_MUL)
    with pytest.raises(HipError):
        eng.matvec(even, xq, y, 1, bias=b, mode=SILU_MUL)
    with pytest.raises(HipError):
        eng.gemm(even, xq, y, 16, bias=b, mode=SILU_MUL)
    with pytest.raises(HipError):
        eng.mm(even, xq, y, 16, bias=b, mode=SILU_MUL)
    with pytest.raises(HipError):
        eng.gemm(odd, xq, y, 16, mode=SILU_MUL)
    eng.matvec(even, xq, y, 1, mode=SILU_MUL)
    eng.gemm(even, xq, y, 16, mode=SILU_MUL)
    torch.cuda.synchronize()
    eng.free(odd)
    eng.free(even)


# ---------------------------------------------------------------------------------------- full-size prefill

@pytest.mark.parametrize("t,m,k", [(F.Q4_K, 14336, 4096), (F.Q4_K, 4096, 14336), (F.IQ4_NL, 14336, 4096),
                                   (F.Q6_K, 4096, 14336), (F.Q8_0, 14336, 4096)])
def test_full_size_prefill_rows(eng, torch_cuda, t, m, k):
    """The BASELINE 8B FFN prefill GEMMs (512 tokens) at full size. Each output row depends only
    on its weight row, so the oracle is run on a sample of rows -- the first and last, rows at the
    kernels' 16/32/128/256-row tile edges and random ones -- against all 512 tokens."""
    n = 512
    raw = synth.weights_np(t, m, k, seed=1500 + t)
    x = synth.activations_np(n, k, seed=1501, outliers=0.01)
    got = run(eng, torch_cuda, t, raw, m, k, x, path="mm")
    rng = np.random.default_rng(1502)
    edges = [0, 1, 15, 16, 31, 32, 127, 128, 255, 256, m // 2, m - 257, m - 33, m - 2, m - 1]
    rows = np.unique(np.concatenate([np.array(edges), rng.integers(0, m, 33)]))
    want = O.matmul(t, raw[rows], len(rows), k, x, n, threads=16)
    assert parity_err(got[:, rows], want) <= PARITY_TOL


@pytest.mark.parametrize("t,m,k", [(F.Q4_K, 14336, 4096), (F.Q4_K, 4096, 14336), (F.Q6_K, 128256, 4096)])
def test_full_size_batch8_rows(eng, torch_cuda, t, m, k):
    """The batch-8 decode products of config 4 at full size (the small-batch kernel on a prepared
    input), the 128256-row Q6_K lm_head included; a sample of rows against the oracle."""
    torch = torch_cuda
    n = 8
    raw = synth.weights_np(t, m, k, seed=1600 + t)
    x = synth.activations_np(n, k, seed=1601)
    w = eng.upload(raw, t, m, k)
    xd = torch.from_numpy(x).cuda()
    xq = torch.empty(eng.act_bytes(n, k), dtype=torch.uint8, device="cuda")
    eng.qact(xd, n, k, F.ACT_KIND[t], xq)
    y = torch.full((n, m), float("nan"), device="cuda")
    eng.matvec_parts([w], [y], n, xq=xq)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    eng.free(w)
    rng = np.random.default_rng(1602)
    rows = np.unique(np.concatenate([np.array([0, 1, 15, 16, 17, m // 2, m - 17, m - 16, m - 1]),
                                     rng.integers(0, m, 55)]))
    want = O.matmul(t, raw[rows], len(rows), k, x, n, threads=16)
    assert parity_err(got[:, rows], want) <= PARITY_TOL
    assert np.isfinite(got).all()


@pytest.mark.parametrize("t", [F.Q4_K, F.Q6_K])
@pytest.mark.parametrize("n,mode", [(5, 0), (20, 1), (8, 2)])
def test_small_batch_many_tiles(eng, torch_cuda, t, n, mode):
    """The small-batch kernel over two fused parts with ragged heights (over 1000 row tiles), one
    or two token tiles, bias and accumulate, and silu(gate)*up."""
    torch = torch_cuda
    k = 512
    heights = [9000, 7778] if mode == 2 else [9000, 7777]
    raws = [synth.weights_np(t, m, k, seed=1700 + i + t) for i, m in enumerate(heights)]
    x = synth.activations_np(n, k, seed=1701 + n, outliers=0.01)
    mats = [eng.upload(r, t, m, k) for r, m in zip(raws, heights)]
    cols = [m // 2 if mode == 2 else m for m in heights]
    y0s = [synth.activations_np(n, c, seed=1702 + c) for c in cols]
    ys = [torch.from_numpy(y0.copy()).cuda() if mode == 1 else torch.full((n, c), float("nan"), device="cuda")
          for y0, c in zip(y0s, cols)]
    biases = [torch.from_numpy(np.linspace(-1, 1, m).astype(np.float32)).cuda() for m in heights] if mode != 2 else None
    xq = torch.empty(eng.act_bytes(n, k), dtype=torch.uint8, device="cuda")
    eng.qact(torch.from_numpy(x).cuda(), n, k, F.ACT_KIND[t], xq)
    if n <= 8:
        eng.matvec_parts(mats, ys, n, xq=xq, biases=biases, mode=mode)
    else:
        for w, y, b in zip(mats, ys, biases):
            eng.mm(w, xq, y, n, bias=b, mode=mode)
    torch.cuda.synchronize()
    for i, (r, m) in enumerate(zip(raws, heights)):
        b = biases[i].cpu().numpy() if biases else None
        want = O.matmul(t, r, m, k, x, n, bias=b, tiled=False)
        if mode == 1:
            want = want + y0s[i]
        if mode == 2:
            want = silu_mul_ref(want)
        assert parity_err(ys[i].cpu().numpy(), want) <= PARITY_TOL
    for w in mats:
        eng.free(w)


@pytest.mark.parametrize("t", [F.Q4_K, F.Q6_K])
@pytest.mark.parametrize("n,m,k", [(7, 16400, 768), (4, 16385, 256), (8, 24576, 1280)])
def test_small_batch_shared_activations(eng, torch_cuda, t, n, m, k):
    """The small-batch products whose launch is large enough for workgroups that stage the tokens'
    activations in LDS once (at most 8 tokens, 256 or more workgroups of four 16-row tiles): odd
    super-block counts (ring steps past the end), a single super-block, and a last workgroup
    whose waves are mostly past the last row tile (16400 and 16385 rows); every row against the
    oracle, with a bias."""
    torch = torch_cuda
    raw = synth.weights_np(t, m, k, seed=1750 + t + n)
    x = synth.activations_np(n, k, seed=1751 + n, outliers=0.01)
    w = eng.upload(raw, t, m, k)
    xq = torch.empty(eng.act_bytes(n, k), dtype=torch.uint8, device="cuda")
    eng.qact(torch.from_numpy(x).cuda(), n, k, F.ACT_KIND[t], xq)
    bias = np.linspace(-2, 2, m).astype(np.float32)
    y = torch.full((n, m), float("nan"), device="cuda")
    eng.matvec_parts([w], [y], n, xq=xq, biases=[torch.from_numpy(bias).cuda()])
    torch.cuda.synchronize()
    want = O.matmul(t, raw, m, k, x, n, bias=bias, threads=16)
    assert parity_err(y.cpu().numpy(), want) <= PARITY_TOL
    eng.free(w)


@pytest.mark.parametrize("t", [F.Q4_K, F.Q6_K])
@pytest.mark.parametrize("n,mode", [(5, 1), (8, 1), (6, 2)])
def test_small_batch_shared_activations_modes(eng, torch_cuda, t, n, mode):
    """The shared-activation workgroups with two fused parts of ragged heights (1027 row tiles, a
    part boundary inside a workgroup), in accumulate mode with biases and in silu(gate)*up mode;
    every row against the oracle."""
    torch = torch_cuda
    k = 1024
    heights = [8210, 8222] if mode == 2 else [8209, 8223]
    raws = [synth.weights_np(t, m, k, seed=1760 + i + t + n) for i, m in enumerate(heights)]
    x = synth.activations_np(n, k, seed=1761 + n, outliers=0.01)
    mats = [eng.upload(r, t, m, k) for r, m in zip(raws, heights)]
    cols = [m // 2 if mode == 2 else m for m in heights]
    y0s = [synth.activations_np(n, c, seed=1762 + c) for c in cols]
    ys = [torch.from_numpy(y0.copy()).cuda() if mode == 1 else torch.full((n, c), float("nan"), device="cuda")
          for y0, c in zip(y0s, cols)]
    biases = [np.linspace(-1, 1, m).astype(np.float32) for m in heights] if mode == 1 else None
    xq = torch.empty(eng.act_bytes(n, k), dtype=torch.uint8, device="cuda")
    eng.qact(torch.from_numpy(x).cuda(), n, k, F.ACT_KIND[t], xq)
    eng.matvec_parts(mats, ys, n, xq=xq, mode=mode,
                     biases=[torch.from_numpy(b).cuda() for b in biases] if biases else None)
    torch.cuda.synchronize()
    for i, (r, m) in enumerate(zip(raws, heights)):
        want = O.matmul(t, r, m, k, x, n, bias=biases[i] if biases else None, threads=16)
        want = want + y0s[i] if mode == 1 else silu_mul_ref(want)
        assert parity_err(ys[i].cpu().numpy(), want) <= PARITY_TOL
    for w in mats:
        eng.free(w)


@pytest.mark.parametrize("t", FMTS)
def test_gemm_unaligned_output(eng, torch_cuda, t):
    """Outputs that are not 16-byte aligned (here one float past an aligned buffer) take the
    per-lane stores of the GEMM's epilogue; the aligned case takes the staged 16-byte stores."""
    torch = torch_cuda
    m, k, n = 1024, 512, 96
    raw = synth.weights_np(t, m, k, seed=1800 + t)
    x = synth.activations_np(n, k, seed=1801)
    w = eng.upload(raw, t, m, k)
    xq = torch.empty(eng.act_bytes(n, k), dtype=torch.uint8, device="cuda")
    eng.qact(torch.from_numpy(x).cuda(), n, k, F.ACT_KIND[t], xq)
    want = O.matmul(t, raw, m, k, x, n, threads=16)
    for off in (0, 1):
        buf = torch.full((n * m + 4,), float("nan"), device="cuda")
        y = buf[off:off + n * m]
        eng.gemm(w, xq, y, n)
        torch.cuda.synchronize()
        assert parity_err(y.view(n, m).cpu().numpy(), want) <= PARITY_TOL
        assert torch.isnan(buf[:off]).all() and torch.isnan(buf[off + n * m:]).all()
    eng.free(w)


# ---------------------------------------------------------------------------------------- the timed paths

TIMED = {
    # bench.py's batch-1 decode step (config 4): fused launches on an f32 input, quantized in-kernel
    "llama8b-qkv": (F.Q4_K, [4096, 1024, 1024], 4096),
    "llama8b-o": (F.Q4_K, [4096], 4096),
    "llama8b-gate-up": (F.Q4_K, [14336, 14336], 4096),
    "llama8b-down": (F.Q4_K, [4096], 14336),
    "llama8b-lm-head": (F.Q6_K, [128256], 4096),
    # config 2 (Qwen3-0.6B decode step)
    "qwen-qkv": (F.Q4_K, [2048, 1024, 1024], 1024),
    "qwen-o": (F.Q4_K, [1024], 2048),
    "qwen-gate-up": (F.Q4_K, [3072, 3072], 1024),
    "qwen-down": (F.Q4_K, [1024], 3072),
    "qwen-lm-head": (F.Q6_K, [151936], 1024),
    # config 1 and config 5's batch-1 products
    "config1-q8_0": (F.Q8_0, [3072], 1024),
    "config5-iq4_nl-up": (F.IQ4_NL, [14336], 4096),
    "config5-q6_k-down": (F.Q6_K, [4096], 14336),
}


@pytest.mark.parametrize("n,prepared", [(1, False), (8, True)])
@pytest.mark.parametrize("workload", list(TIMED))
def test_timed_decode_paths(eng, torch_cuda, workload, n, prepared):
    """Every product the bench times, at its full shape and through the same entry point and
    kernel choice: hkhip_matvec_parts on the f32 input (batch 1; the kernel quantizes it) or on an
    input prepared by hkhip_qact (batch 8, as the batch-8 step runs it), with the bench's fusion
    of parts. Tall matrices are checked on a sample of rows (each output row depends only on its
    weight row): the first and last, rows around 16/64-row edges and random ones."""
    torch = torch_cuda
    t, heights, k = TIMED[workload]
    outl = 0.01 if workload.startswith("config5") else 0.0
    x = synth.activations_np(n, k, seed=2200 + n, outliers=outl)
    raws = [synth.weights_np(t, m, k, seed=2300 + i + m) for i, m in enumerate(heights)]
    mats = [eng.upload(r, t, m, k) for r, m in zip(raws, heights)]
    ys = [torch.full((n, m), float("nan"), device="cuda") for m in heights]
    xd = torch.from_numpy(x).cuda()
    if prepared:
        xq = torch.empty(eng.act_bytes(n, k), dtype=torch.uint8, device="cuda")
        eng.qact(xd, n, k, F.ACT_KIND[t], xq)
        eng.matvec_parts(mats, ys, n, xq=xq)
    else:
        eng.matvec_parts(mats, ys, n, x=xd)
    torch.cuda.synchronize()
    for w in mats:
        eng.free(w)
    rng = np.random.default_rng(2400)
    for r, m, y in zip(raws, heights, ys):
        got = y.cpu().numpy()
        assert np.isfinite(got).all()
        if m > 4096:
            rows = np.unique(np.concatenate([np.array([0, 1, 15, 16, 63, 64, 65, m // 2, m - 65, m - 64, m - 17,
                                                       m - 16, m - 2, m - 1]), rng.integers(0, m, 64)]))
        else:
            rows = np.arange(m)
        want = O.matmul(t, r[rows], len(rows), k, x, n, tiled=False, threads=16)
        assert parity_err(got[:, rows], want) <= PARITY_TOL, workload


def test_engine_from_another_thread(torch_cuda):
    """An engine created and loaded on one thread, then driven from a worker thread, as hk's
    server does (tests/test_gpu.zig:446-478 checkOtherThread): every entry point makes the
    engine's device current, so upload, qact, the products and sync work there."""
    import threading

    from hk_amd import Engine

    torch = torch_cuda
    t, m, k = F.Q4_K, 300, 1024
    raw = synth.weights_np(t, m, k, seed=2500)
    raw2 = synth.weights_np(F.Q8_0, 64, k, seed=2501)
    x = synth.activations_np(12, k, seed=2502)
    e = Engine(0)  # its own stream: nothing here depends on torch's stream
    w = e.upload(raw, t, m, k)
    xd = torch.from_numpy(x).cuda()
    ys = {n: torch.full((n, m), float("nan"), device="cuda") for n in (1, 12)}
    y2 = torch.full((1, 64), float("nan"), device="cuda")
    torch.cuda.synchronize()
    out = {}

    def job():
        try:
            w2 = e.upload(raw2, F.Q8_0, 64, k)
            xq = torch.empty(e.act_bytes(12, k), dtype=torch.uint8, device="cuda")
            e.qact(xd, 12, k, F.ACT_Q8K, xq)
            e.mm(w, xq, ys[12], 12)
            e.matvec_parts([w], [ys[1]], 1, x=xd[:1])
            e.matvec_parts([w2], [y2], 1, x=xd[:1])
            e.sync()
            e.free(w2)
            out["ok"] = True
        except Exception as exc:  # reported by the main thread
            out["err"] = exc

    th = threading.Thread(target=job)
    th.start()
    th.join()
    assert out.get("ok"), out.get("err")
    for n, y in ys.items():
        assert parity_err(y.cpu().numpy(), O.matmul(t, raw, m, k, x[:n], n)) <= PARITY_TOL
    assert parity_err(y2.cpu().numpy(), O.matmul(F.Q8_0, raw2, 64, k, x[:1], 1)) <= PARITY_TOL
    e.close()


@pytest.mark.parametrize("t", [F.Q5_K, F.Q4_0, F.Q4_1, F.IQ4_XS])
@pytest.mark.parametrize("n", [9, 12, 16])
def test_mm_tall_break_even(eng, torch_cuda, t, n):
    """hkhip_mm on matrices of at least 8192 rows switches these formats to the GEMM from 9 tokens:
    the ragged 32-token tile at 9-16 tokens, with bias and accumulate."""
    m, k = 9000, 4096
    raw = synth.weights_np(t, m, k, seed=2600 + t)
    x = synth.activations_np(n, k, seed=2601 + n)
    bias = np.linspace(-1, 1, m).astype(np.float32)
    y0 = synth.activations_np(n, m, seed=2602)
    got = run(eng, torch_cuda, t, raw, m, k, x, path="mm", bias=bias, mode=1, y0=y0)
    want = O.matmul(t, raw, m, k, x, n, bias=bias, threads=16) + y0
    assert parity_err(got, want) <= PARITY_TOL


# ---------------------------------------------------------------------------------------- fused RMS norm

@pytest.mark.parametrize("t", FMTS)
@pytest.mark.parametrize("n,k", [(1, 1024), (1, 4096), (3, 2048), (8, 4096), (1, 14336), (2, 3072)])
def test_matvec_parts_rmsnorm(eng, torch_cuda, t, n, k):
    """hkhip_matvec_parts_rmsnorm: rmsnorm(x) * w (ops.zig:10-29) fused into the products' input
    quantization, q/k/v-style parts with biases, against the oracle's products of the CPU norm."""
    from oracle.net_oracle import rms_norm

    torch = torch_cuda
    heights = [96, 40]
    raws = [synth.weights_np(t, m, k, seed=2700 + i + t) for i, m in enumerate(heights)]
    x = synth.activations_np(n, k, seed=2701 + n, outliers=0.01) * 3.0
    w = (1.0 + 0.1 * np.random.default_rng(2702).standard_normal(k)).astype(np.float32)
    eps = 1e-6
    mats = [eng.upload(r, t, m, k) for r, m in zip(raws, heights)]
    ys = [torch.full((n, m), float("nan"), device="cuda") for m in heights]
    biases = [torch.from_numpy(np.linspace(-1, 1, m).astype(np.float32)).cuda() for m in heights]
    eng.matvec_parts_rmsnorm(mats, ys, n, torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), eps, biases=biases)
    torch.cuda.synchronize()
    xb = np.stack([rms_norm(x[i], w, eps) for i in range(n)])
    for r, m, y, b in zip(raws, heights, ys, biases):
        want = O.matmul(t, r, m, k, xb, n, bias=b.cpu().numpy(), tiled=False)
        assert parity_err(y.cpu().numpy(), want) <= PARITY_TOL
    for mm in mats:
        eng.free(mm)


def test_matvec_parts_rmsnorm_silu_and_limits(eng, torch_cuda):
    from hk_amd import HipError
    from oracle.net_oracle import rms_norm

    torch = torch_cuda
    t, m, k, n = F.Q4_K, 2 * 200, 4096, 2
    raw = synth.weights_np(t, m, k, seed=2710)
    x = synth.activations_np(n, k, seed=2711)
    w = (1.0 + 0.1 * np.random.default_rng(2712).standard_normal(k)).astype(np.float32)
    mat = eng.upload(raw, t, m, k)
    y = torch.full((n, m // 2), float("nan"), device="cuda")
    xd, wd = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
    eng.matvec_parts_rmsnorm([mat], [y], n, xd, wd, 1e-5, mode=SILU_MUL)
    torch.cuda.synchronize()
    xb = np.stack([rms_norm(x[i], w, 1e-5) for i in range(n)])
    want = silu_mul_ref(O.matmul(t, raw, m, k, xb, n, tiled=False))
    assert parity_err(y.cpu().numpy(), want) <= PARITY_TOL
    x9 = torch.zeros(9, k, device="cuda")
    with pytest.raises(HipError) as e:
        eng.matvec_parts_rmsnorm([mat], [torch.zeros(9, m, device="cuda")], 9, x9, wd, 1e-5)
    assert e.value.code == -2
    eng.free(mat)
