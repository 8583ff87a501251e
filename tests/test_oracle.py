"""Pins of the CPU oracle (CPU only; no GPU).

The oracle restates hk's CPU kernels in C. Each part is pinned by something other than its own
formula:
  decoders     hk's fixtures, written by the gguf reference decoder (tools/gen_quant_fixtures.py),
               bit for bit up to the sign of zero
  scale unpack the word trick of vecdot.zig:461-474 against scaleMinK4 (dequant.zig:166-175) on
               every possible byte pattern of each scale position
  quantizers   closed-form invariants (|q| <= 127, the extreme element hits +-127, d*q within
               d/2 of x, s / bsums are the sums of q, the all-zero block, first-index ties)
  dots         an independent float64 restatement from the decoded weights and the dequantized
               activations (d * q), which is algebraically the integer dot, to 1e-5 of the terms;
               and hk's own bound against the float decode-dot (test_quant.zig:161)
  GEMM path    equal to the row dots within 1e-4 (test_quant.zig:326), 37 rows x 11 tokens
"""
from __future__ import annotations

import numpy as np
import pytest

from hk_amd import formats as F
from hk_amd import synth
from oracle import oracle as O
from tests.helpers import load_fixture, tie_rows

FMTS = [F.Q8_0, F.Q4_K, F.Q6_K, F.IQ4_NL, F.Q4_0, F.Q4_1, F.Q5_0, F.Q5_1, F.Q5_K, F.IQ4_XS]
FIXTURES = F.NAMES
GGML_TYPE = {F.Q8_0: 8, F.Q4_K: 12, F.Q6_K: 14, F.IQ4_NL: 20, F.Q4_0: 2, F.Q4_1: 3, F.Q5_0: 6, F.Q5_1: 7,
             F.Q5_K: 13, F.IQ4_XS: 23, F.Q2_K: 10, F.Q3_K: 11, F.IQ2_XXS: 16, F.IQ2_XS: 17, F.IQ3_XXS: 18,
             F.IQ1_S: 19, F.IQ3_S: 21, F.IQ2_S: 22, F.IQ1_M: 29, F.TQ1_0: 34, F.TQ2_0: 35, F.MXFP4: 39, F.NVFP4: 40}


@pytest.fixture(scope="module", autouse=True)
def built():
    O.build()


# ------------------------------------------------------------------------------------ decoders

@pytest.mark.parametrize("t", FMTS + list(F.FALLBACK))
def test_fixture_geometry(t):
    fx = load_fixture(FIXTURES[t])
    assert fx["ggml_type"] == GGML_TYPE[t]
    assert (fx["block_elems"], fx["block_bytes"]) == F.INFO[t]
    assert (O.block_elems(t), O.block_bytes(t)) == F.INFO[t]


@pytest.mark.parametrize("t", FMTS + list(F.FALLBACK))
def test_decoders_match_reference_fixtures(t):
    fx = load_fixture(FIXTURES[t])
    k = fx["blocks_per_row"] * fx["block_elems"]
    got = np.stack([O.dequantize(t, fx["raw"][r], k) for r in range(fx["rows"])])
    want = fx["expected"]
    assert np.array_equal(got, want)  # exact values (0.0 == -0.0)
    diff = got.view(np.uint32) != want.view(np.uint32)
    # hk's q6_k decoder computes d * f32(scale * q), which is -0.0 for a negative d and q = 0;
    # gguf writes +0.0 there. Every other bit agrees.
    assert np.all(got[diff] == 0.0)
    if t != F.Q6_K:
        assert not diff.any()


def test_dequantize_rejects_wrong_lengths():
    """dequantizeRow refuses partial blocks (test_quant.zig 'decoding rejects wrong lengths')."""
    with pytest.raises(ValueError):
        O.dequantize(F.Q8_0, np.zeros(33, np.uint8), 32)
    with pytest.raises(ValueError):
        O.dequantize(F.Q8_0, np.zeros(34, np.uint8), 31)
    with pytest.raises(ValueError):
        O.dequantize(0x22, np.zeros(34, np.uint8), 32)


@pytest.mark.parametrize("t", FMTS)
def test_decode_closed_forms_on_constructed_blocks(t):
    """Hand-built blocks whose values follow from the format definition alone."""
    if t == F.Q8_0:
        b = np.zeros(34, np.uint8)
        b[0:2] = np.array([0.5], np.float16).view(np.uint8)
        b[2:34] = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
        assert np.array_equal(O.dequantize(t, b, 32), np.arange(-16, 16) * 0.5)
    elif t == F.IQ4_NL:
        b = np.zeros(18, np.uint8)
        b[0:2] = np.array([2.0], np.float16).view(np.uint8)
        b[2:18] = (np.arange(16) | ((15 - np.arange(16)) << 4)).astype(np.uint8)
        want = 2.0 * np.array(F.KVALUES_IQ4NL + F.KVALUES_IQ4NL[::-1], np.float32)
        assert np.array_equal(O.dequantize(t, b, 32), want)
    elif t == F.Q4_K:
        b = np.zeros(144, np.uint8)
        b[0:2] = np.array([1.0], np.float16).view(np.uint8)   # d
        b[2:4] = np.array([0.25], np.float16).view(np.uint8)  # dmin
        # sub-block j: scale j + 1, min 2j (all below 16, so only the low 4 bits are used)
        for j in range(8):
            sc, mn = j + 1, 2 * j
            if j < 4:
                b[4 + j] = sc
                b[8 + j] = mn
            else:
                b[8 + j] = sc | (mn << 4)
        b[16:144] = 0x53  # low nibble 3, high nibble 5
        got = O.dequantize(t, b, 256)
        for j in range(8):
            nib = 3 if j % 2 == 0 else 5
            want = (j + 1) * 1.0 * nib - 0.25 * (2 * j)
            assert np.all(got[32 * j:32 * j + 32] == np.float32(want))
    elif t in (F.Q4_0, F.Q4_1, F.Q5_0, F.Q5_1):
        # ggml's block definitions: byte j holds weight j (low nibble) and j + 16 (high nibble);
        # Q5 takes bit j of the little-endian qh word as weight j's fifth bit.
        five, has_m = t in (F.Q5_0, F.Q5_1), t in (F.Q4_1, F.Q5_1)
        nb = F.INFO[t][1]
        b = np.zeros(nb, np.uint8)
        b[0:2] = np.array([0.5], np.float16).view(np.uint8)
        off = 2
        if has_m:
            b[2:4] = np.array([-1.25], np.float16).view(np.uint8)
            off = 4
        qh = 0xA5C3F00F
        if five:
            b[off:off + 4] = np.array([qh], "<u4").view(np.uint8)
            off += 4
        b[off:off + 16] = (np.arange(16) | ((15 - np.arange(16)) << 4)).astype(np.uint8)
        u = [j if j < 16 else 31 - j for j in range(32)]
        if five:
            u = [u[j] + 16 * ((qh >> j) & 1) for j in range(32)]
        zp = {F.Q4_0: 8, F.Q5_0: 16}.get(t, 0)
        want = [np.float32(uj) * np.float32(0.5) + np.float32(-1.25) if has_m else np.float32(uj - zp) * np.float32(0.5)
                for uj in u]
        assert np.array_equal(O.dequantize(t, b, 32), np.array(want, np.float32))
    elif t == F.Q5_K:
        # Q4_K's block with qh[32] before qs: weight l of chunk c's low (high) half takes bit 2c
        # (2c + 1) of qh[l] as its fifth bit.
        b = np.zeros(176, np.uint8)
        b[0:2] = np.array([1.0], np.float16).view(np.uint8)
        b[2:4] = np.array([0.25], np.float16).view(np.uint8)
        for j in range(8):
            sc, mn = j + 1, 2 * j
            if j < 4:
                b[4 + j], b[8 + j] = sc, mn
            else:
                b[8 + j] = sc | (mn << 4)
        b[16:48] = (np.arange(32) * 37 % 256).astype(np.uint8)
        b[48:176] = 0x53
        got = O.dequantize(t, b, 256)
        for c in range(4):
            for half in range(2):
                j = 2 * c + half
                for l in range(32):
                    u = (3 if half == 0 else 5) + 16 * ((int(b[16 + l]) >> j) & 1)
                    assert got[64 * c + 32 * half + l] == np.float32(np.float32(j + 1) * np.float32(u) - np.float32(0.25 * 2 * j))
    elif t == F.IQ4_XS:
        # d, scales_h (2 bits per sub-block), scales_l (4 bits per sub-block), 16 B of indices per
        # sub-block; sub-block scale = 6-bit value - 32.
        b = np.zeros(136, np.uint8)
        b[0:2] = np.array([0.5], np.float16).view(np.uint8)
        ls6 = [0, 63, 32, 31, 1, 40, 17, 50]
        sh = sum((v >> 4) << (2 * ib) for ib, v in enumerate(ls6))
        b[2:4] = np.array([sh], "<u2").view(np.uint8)
        for ib, v in enumerate(ls6):
            b[4 + ib // 2] |= (v & 15) << (4 * (ib % 2))
        b[8:136] = np.tile((np.arange(16) | ((15 - np.arange(16)) << 4)).astype(np.uint8), 8)
        got = O.dequantize(t, b, 256)
        kv = F.KVALUES_IQ4NL
        for ib, v in enumerate(ls6):
            dl = np.float32(0.5) * np.float32(v - 32)
            want = [dl * np.float32(kv[j]) for j in range(16)] + [dl * np.float32(kv[15 - j]) for j in range(16)]
            assert np.array_equal(got[32 * ib:32 * ib + 32], np.array(want, np.float32))
    else:  # Q6_K
        b = np.zeros(210, np.uint8)
        b[208:210] = np.array([0.5], np.float16).view(np.uint8)
        b[192:208] = np.arange(-8, 8, dtype=np.int8).view(np.uint8)  # scale per 16
        b[0:128] = 0x21   # low 4 bits: 1 (ql low nibble), 2 (ql high nibble)
        b[128:192] = 0xE4  # high 2 bits per quarter: 0, 1, 2, 3
        got = O.dequantize(t, b, 256)
        for half in range(2):
            for part, (low, hi2) in enumerate([(1, 0), (1, 1), (2, 2), (2, 3)]):
                q = (low | (hi2 << 4)) - 32
                for l in range(32):
                    g = 8 * half + 2 * part + l // 16
                    assert got[128 * half + 32 * part + l] == np.float32(0.5 * ((g - 8) * q))


def test_scale_unpack_word_trick_matches_scale_min_k4():
    """scalesMinsK4 (vecdot.zig:461-474) and scaleMinK4 (dequant.zig:166-175) agree on every
    byte value at every one of the 12 positions, with the other bytes random."""
    rng = np.random.default_rng(5)
    for pos in range(12):
        for v in range(256):
            p = rng.integers(0, 256, 12, dtype=np.uint8)
            p[pos] = v
            sc, mn = O.scales_mins_words(p)
            for j in range(8):
                assert (sc[j], mn[j]) == O.scale_min_k4(j, p)


# ------------------------------------------------------------------------------------ quantizers

def _round_half_away(v):
    a = np.abs(v.astype(np.float64))
    f = np.floor(a)
    return np.sign(v) * (f + (a - f >= 0.5))


def test_quantize_a8_invariants():
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, 32 * 64).astype(np.float32)
    x[32:64] = 0.0                        # zero block
    x[64:96] = rng.normal(0, 1e-30, 32)   # denormal-range block
    x[96:128] *= 1e4
    blocks = O.quantize_a8(x)
    for b, blk in enumerate(blocks):
        v = x[32 * b:32 * b + 32]
        q = blk["qs"].astype(np.int64)
        amax = np.max(np.abs(v))
        assert blk["d"] == np.float32(amax) / np.float32(127.0)
        assert blk["s"] == q.sum()
        assert np.all(np.abs(q) <= 127)
        if amax == 0:
            assert np.all(q == 0) and blk["d"] == 0
            continue
        i = int(np.argmax(np.abs(v)))
        assert abs(q[i]) == 127 and np.sign(q[i]) == np.sign(v[i])
        # q = round_half_away(x * (1/d)) in f32 arithmetic
        idv = np.float32(1.0) / np.float32(blk["d"])
        assert np.array_equal(q, _round_half_away(v * idv))
        assert np.all(np.abs(v - blk["d"] * q) <= blk["d"] * 0.5 * (1 + 1e-5) + 1e-37)


def test_quantize_q8k_invariants():
    rng = np.random.default_rng(2)
    x = rng.normal(0, 1, 256 * 16).astype(np.float32)
    x[256:512] = 0.0
    x[512 + 10], x[512 + 200] = -9.0, 9.0   # tie on |x|: the first (negative) one wins
    x[768 + 10], x[768 + 200] = 9.0, -9.0
    x[1024:1280] *= 1e-30
    blocks = O.quantize_q8k(x)
    for b, blk in enumerate(blocks):
        v = x[256 * b:256 * b + 256]
        q = blk["qs"].astype(np.int64)
        assert np.array_equal(blk["bsums"], q.reshape(16, 16).sum(axis=1))
        if np.max(np.abs(v)) == 0:
            assert np.all(q == 0) and blk["d"] == 0 and np.all(blk["bsums"] == 0)
            continue
        i = int(np.argmax(np.abs(v)))  # numpy's argmax returns the first maximum
        assert q[i] == -127            # iscale * max = -127
        assert np.sign(blk["d"]) == -np.sign(v[i])
        assert np.all(q <= 127) and np.all(q >= -128)
        err = np.abs(v - blk["d"] * q)
        clamped = q == 127
        assert np.all(err[~clamped] <= abs(blk["d"]) * 0.5 * (1 + 1e-5) + 1e-37)
    assert blocks[2]["d"] > 0 and blocks[3]["d"] < 0  # the tie rule: first index sets the sign


def test_quantizers_round_ties_half_away():
    """Tie values k + 0.5 at scale exactly 1 (tests.helpers.tie_rows): both quantizers must round
    them away from zero, as Zig's @round does (vecdot.zig:141, 172); rint would fail here."""
    x, q = tie_rows(512)
    a8 = O.quantize_a8(x[0])
    assert np.all(a8["d"] == 1.0)
    assert np.array_equal(a8["qs"].astype(np.int64).ravel(), q[0])
    assert np.array_equal(a8["s"], q[0].reshape(-1, 32).sum(axis=1))
    qk = O.quantize_q8k(x[0])
    assert np.all(qk["d"] == 1.0)
    assert np.array_equal(qk["qs"].astype(np.int64).ravel(), q[0])
    assert np.array_equal(qk["bsums"].astype(np.int64).ravel(), q[0].reshape(-1, 16).sum(axis=1))


# ------------------------------------------------------------------------------------ dots

def _decoded_act(t, x):
    """Dequantized activations d * q, the value the integer dot multiplies by."""
    if F.ACT_KIND[t] == F.ACT_A8:
        a = O.quantize_a8(x)
        return (a["d"][:, None].astype(np.float64) * a["qs"].astype(np.float64)).ravel(), a
    a = O.quantize_q8k(x)
    return (a["d"][:, None].astype(np.float64) * a["qs"].astype(np.float64)).ravel(), a


@pytest.mark.parametrize("t", FMTS)
def test_dot_equals_float64_restatement(t):
    """The integer dot equals sum_k w_k * (d_a q_k) (exact algebra) up to f32 rounding."""
    rng = np.random.default_rng(0xD07)
    k = 1024
    raw = synth.weights_np(t, 6, k, seed=9 + t)
    for trial in range(4):
        x = rng.normal(0, 1, k).astype(np.float32)
        if trial == 3:
            x[rng.random(k) < 0.01] = 20.0
        xa, act = _decoded_act(t, x)
        for r in range(raw.shape[0]):
            w = O.dequantize(t, raw[r], k).astype(np.float64)
            want = float(np.sum(w * xa))
            terms = float(np.sum(np.abs(w * xa)))
            got = O.dot_row(t, raw[r], act)
            assert abs(got - want) <= 1e-5 * terms + 1e-6


@pytest.mark.parametrize("t", FMTS)
def test_dot_within_reference_bound_on_fixtures(t):
    """hk's own check (test_quant.zig:121-194): integer dot vs float64 decode-dot of the f32
    activations, within 0.01 * sum|terms| + 1e-4."""
    fx = load_fixture(FIXTURES[t])
    k = fx["blocks_per_row"] * fx["block_elems"]
    rng = np.random.default_rng(0xD07)
    for _ in range(8):
        x = (rng.random(k) * 2 - 1).astype(np.float32)
        _, act = _decoded_act(t, x)
        for r in range(fx["rows"]):
            w = O.dequantize(t, fx["raw"][r], k).astype(np.float64)
            want = float(np.sum(w * x))
            tol = 0.01 * float(np.sum(np.abs(w * x))) + 1e-4
            assert abs(O.dot_row(t, fx["raw"][r], act) - want) <= tol


@pytest.mark.parametrize("t", FMTS)
def test_gemm_path_equals_row_dots(t):
    """gemm.tiles equals vecdot single dots (test_quant.zig:281-359): 37 rows from the fixture
    rows, 11 tokens, bias i % 5, within 1e-4 * max(1, |want|)."""
    fx = load_fixture(FIXTURES[t])
    k = fx["blocks_per_row"] * fx["block_elems"]
    raw = np.stack([fx["raw"][r % fx["rows"]] for r in range(37)])
    x = np.random.default_rng(0x6E33).uniform(-1, 1, (11, k)).astype(np.float32)
    bias = (np.arange(37) % 5).astype(np.float32)
    tiled = O.matmul(t, raw, 37, k, x, 11, bias=bias, tiled=True)
    rows = O.matmul(t, raw, 37, k, x, 11, bias=bias, tiled=False)
    assert np.all(np.abs(tiled - rows) <= 1e-4 * np.maximum(1.0, np.abs(rows)))


def test_matmul_dispatch_and_threads():
    """n >= 8 takes the tiled path (matmul.zig:18); threads do not change results."""
    t, m, k = F.Q4_K, 40, 512
    raw = synth.weights_np(t, m, k, seed=3)
    for n in (7, 8):
        x = synth.activations_np(n, k, seed=4)
        y1 = O.matmul(t, raw, m, k, x, n, threads=1)
        y4 = O.matmul(t, raw, m, k, x, n, threads=4)
        assert np.array_equal(y1, y4)
        assert np.array_equal(y1, O.matmul(t, raw, m, k, x, n, tiled=(n >= 8)))


# ------------------------------------------------------------------------------------ CPU baseline

def test_simd_baseline_levels_match_oracle():
    """hk's SIMD decode kernel (the bench's CPU baseline) at every instruction-set level this
    processor runs gives the oracle's Q4_K matvec bit for bit: the integer dot primitive has one
    exact definition (isa.zig:57-88) and the lanes are summed in the same order."""
    m, k = 77, 2048
    raw = synth.weights_np(F.Q4_K, m, k, seed=41)
    x = synth.activations_np(1, k, seed=42, outliers=0.01)
    want = O.matmul(F.Q4_K, raw, m, k, x, 1, tiled=False)[0]
    ran = []
    for name in O.SIMD_LEVELS:
        lv = O.simd_level(name)
        if lv < 0:
            continue
        got = O.matvec_q4k_simd(raw, m, k, x, threads=3, level=lv)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), name
        ran.append(name)
    assert "generic" in ran and O.simd_level_name(O.simd_level()) == ran[0]


def test_net_oracle_cache_consistency():
    """The CPU network restatement gives the same last-token logits whether a sequence runs as one
    prefill or token by token (its K/V cache carries the earlier positions), and the causal mask
    makes a prefix's logits independent of what follows."""
    from hk_amd.net import Config
    from oracle.net_oracle import Oracle

    cfg = Config(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=256, vocab=128, max_ctx=32)
    model = synth.model_np(cfg, F.Q4_K, seed=77, out_fmt=F.Q6_K, embd_fmt=F.Q8_0)
    toks = np.random.default_rng(78).integers(0, cfg.vocab, 9)
    whole = Oracle(cfg, model).forward(toks, 0)
    step = Oracle(cfg, model)
    for i, tk in enumerate(toks):
        last = step.forward([tk], i)
    assert np.allclose(whole, last, rtol=0, atol=1e-4 * np.abs(whole).max())
    part = Oracle(cfg, model)
    part.forward(toks[:5], 0)
    assert np.allclose(part.forward(toks[5:], 5), whole, rtol=0, atol=1e-4 * np.abs(whole).max())


def test_net_oracle_items_of_several_sequences():
    """The items form of the CPU network restatement: a pass mixing three sequences (a prefill of one
    beside single tokens of the others) leaves every item's hidden state as running that sequence
    alone does; logits of chosen rows match each sequence's own last-token logits; a sequence's
    released cache starts empty again; the leading layers run from the embeddings, then the rest
    from the handed-over hidden states, give the whole pass (the partial-offload split)."""
    from hk_amd.net import Config
    from oracle.net_oracle import Oracle

    cfg = Config(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=256, vocab=128, max_ctx=32)
    model = synth.model_np(cfg, F.Q4_K, seed=79, out_fmt=F.Q6_K, embd_fmt=F.Q8_0, qk_norm=True)
    rng = np.random.default_rng(80)
    ta, tb, tc = (rng.integers(0, cfg.vocab, k) for k in (6, 5, 7))
    solo = {}
    for name, toks in (("a", ta), ("b", tb), ("c", tc)):
        o = Oracle(cfg, model)
        o.forward(toks[:-1], 0) if len(toks) > 1 else None
        solo[name] = o.forward(toks[-1:], len(toks) - 1)
    mixed = Oracle(cfg, model)
    mixed.forward_items([("a", int(t), i) for i, t in enumerate(ta[:3])] + [("b", int(tb[0]), 0)])
    items = [("b", int(t), i + 1) for i, t in enumerate(tb[1:])] + [("a", int(t), i + 3) for i, t in enumerate(ta[3:])] + \
        [("c", int(t), i) for i, t in enumerate(tc)]
    mixed.forward_items(items)
    last = {"b": len(tb) - 2, "a": len(tb) - 2 + len(ta) - 3, "c": len(items) - 1}
    rows = mixed.logits_rows([last["a"], last["b"], last["c"]])
    for r, name in enumerate("abc"):
        want = solo[name]
        assert np.allclose(rows[r], want, rtol=0, atol=1e-5 * np.abs(want).max()), name
    mixed.release("a")
    fresh = mixed.forward_items([("a", int(t), i) for i, t in enumerate(tc)])
    assert np.allclose(mixed.logits_rows([len(tc) - 1])[0], solo["c"], rtol=0, atol=1e-5 * np.abs(solo["c"]).max())
    whole = Oracle(cfg, model).forward_items([(0, int(t), i) for i, t in enumerate(tc)])
    split = Oracle(cfg, model)
    h = split.forward_items([(0, int(t), i) for i, t in enumerate(tc)], layers=1)
    h = split.forward_items([(0, int(t), i) for i, t in enumerate(tc)], hidden=h, first=1)
    assert np.array_equal(h, whole) and np.array_equal(fresh, whole)


def test_net_oracle_quantization_sensitivity():
    """Why the whole-network device tests compare logits within 2e-2 of the largest (with cosine >=
    0.9999, the reference's own device criterion) rather than 1e-3: every product requantizes its
    input (quantizeA8 / quantizeQ8K), so moving the embeddings by one ulp, far less than any
    summation-order difference, flips roundings and moves the CPU restatement's own last-token
    logits by more than 1e-3 of the largest on the test models (measured 7.7e-3 and 1.0e-2 here)."""
    from hk_amd.net import Config
    from oracle.net_oracle import Oracle

    cfg = Config(dim=512, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=128, ffn_dim=768, vocab=400, max_ctx=64,
                 rope_neox=False, rope_base=5e5, rms_eps=1e-5)
    worst = 0.0
    for bias in (True, False):
        model = synth.model_np(cfg, F.Q8_0, seed=4010, out_fmt=F.Q8_0, embd_fmt=F.Q4_K, qk_norm=False, bias=bias)
        toks = np.random.default_rng(4100).integers(0, cfg.vocab, 40)
        items = [(0, int(t), i) for i, t in enumerate(toks)]
        a, b = Oracle(cfg, model), Oracle(cfg, model)
        h = a.embed(toks)
        a.forward_items(items, hidden=h)
        b.forward_items(items, hidden=np.nextafter(h, np.float32(np.inf)).astype(np.float32))
        la, lb = a.logits_rows([39])[0], b.logits_rows([39])[0]
        worst = max(worst, float(np.abs(la - lb).max() / np.abs(la).max()))
    assert 1e-3 < worst < 2e-2, worst


# ------------------------------------------------------------------------------------ float-decode formats

def test_fallback_decoder_closed_forms():
    """Hand-built blocks whose values follow from the format definitions alone."""
    # TQ2_0: 2-bit codes 0..3 mean -1, 0, 1, 2 (hk: q - 1) times d = 1.0 (f16 0x3C00).
    b = np.zeros(66, np.uint8)
    b[0:64] = 0b11100100  # codes 0, 1, 2, 3 in the four 2-bit fields of every byte
    b[64:66] = [0x00, 0x3C]
    got = O.dequantize(F.TQ2_0, b, 256)
    want = np.concatenate([np.full(32, c - 1.0) for _ in range(2) for c in range(4)])
    assert np.array_equal(got, want)
    # MXFP4: E8M0 exponent 128 halves to 2^0 = 1; nibbles index the doubled E2M1 table.
    b = np.zeros(17, np.uint8)
    b[0] = 128
    b[1:17] = np.arange(16, dtype=np.uint8) | (np.arange(16, dtype=np.uint8)[::-1] << 4)
    fp4 = np.array([0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12], np.float32)
    assert np.array_equal(O.dequantize(F.MXFP4, b, 32), np.concatenate([fp4, fp4[::-1]]))
    # NVFP4: E4M3 scale 0x38 (exponent 7, mantissa 0) is 1.0, halved to 0.5.
    b = np.zeros(36, np.uint8)
    b[0:4] = 0x38
    b[4:36] = 0x71  # low nibble 1 (value 1), high nibble 7 (value 12)
    got = O.dequantize(F.NVFP4, b, 64).reshape(4, 2, 8)
    assert np.all(got[:, 0] == 0.5) and np.all(got[:, 1] == 6.0)
    # TQ1_0: every base-3 digit 0 decodes to -1, so an all-zero block with d = 1 is all -1.
    b = np.zeros(54, np.uint8)
    b[52:54] = [0x00, 0x3C]
    assert np.array_equal(O.dequantize(F.TQ1_0, b, 256), np.full(256, -1.0, np.float32))


@pytest.mark.parametrize("t", list(F.FALLBACK))
def test_fallback_products_use_hks_activation_kind(t):
    """The float-decode formats' products take the activation form vecdot.zig:185-191 assigns
    (Q8K for the K and IQ/TQ families, A8 for MXFP4, f32 for NVFP4): the oracle's product equals
    the decoded weights times the activations quantized that way, and differs from the other ways."""
    m, k, n = 9, 512, 3
    raw = synth.weights_np(t, m, k, seed=50 + t)
    x = synth.activations_np(n, k, seed=51)
    w = np.stack([O.dequantize(t, raw[r], k) for r in range(m)]).astype(np.float64)

    def acts(kind):
        if kind == F.ACT_F32:
            return x.astype(np.float64)
        out = []
        for i in range(n):
            a = O.quantize_q8k(x[i]) if kind == F.ACT_Q8K else O.quantize_a8(x[i])
            out.append((a["d"][:, None].astype(np.float64) * a["qs"]).ravel())
        return np.stack(out)

    got = O.matmul(t, raw, m, k, x, n)
    for kind in (F.ACT_A8, F.ACT_Q8K, F.ACT_F32):
        want = acts(kind) @ w.T
        err = np.max(np.abs(got - want)) / np.max(np.abs(want))
        if kind == F.ACT_KIND[t]:
            assert err <= 1e-6
        else:
            assert err > 1e-4


def test_net_oracle_pieces_closed_forms():
    """Closed forms of the CPU network restatement's pieces: RMS norm of a constant vector is
    the weights times sign(c) / sqrt(1 + eps / c^2); RoPE at position 0 is the identity and at any
    position rotates each (i, i + half) or (2i, 2i + 1) pair by pos * base^(-2i/d), keeping its
    length; attention over a single position returns that position's value row."""
    from hk_amd.net import Config
    from oracle.net_oracle import Oracle, rms_norm

    w = np.linspace(0.5, 1.5, 64).astype(np.float32)
    for c in (3.0, -0.25):
        got = rms_norm(np.full(64, c, np.float32), w, 1e-6)
        assert np.allclose(got, w * np.sign(c) / np.sqrt(1 + 1e-6 / c ** 2), rtol=1e-6)
    for neox in (True, False):
        cfg = Config(dim=64, n_layers=1, n_heads=1, n_kv_heads=1, head_dim=64, ffn_dim=256, vocab=16, max_ctx=8,
                     rope_neox=neox, rope_base=10000.0)
        model = synth.model_np(cfg, F.Q8_0, seed=5)
        o = Oracle(cfg, model)
        v = np.random.default_rng(6).standard_normal(64).astype(np.float32)
        assert np.array_equal(o._rope(v, 0), v)
        r = o._rope(v, 5)
        i0, i1 = (np.arange(32), np.arange(32) + 32) if neox else (np.arange(0, 64, 2), np.arange(1, 64, 2))
        ang = 5 * 10000.0 ** (-2 * np.arange(32) / 64)
        want0 = v[i0] * np.cos(ang) - v[i1] * np.sin(ang)
        assert np.allclose(r[i0], want0, atol=1e-5)
        assert np.allclose(np.hypot(r[i0], r[i1]), np.hypot(v[i0], v[i1]), rtol=1e-5)
        # one token: its attention output is its own value row (f16 cache)
        o.forward([3], 0)
        raw, t = model["layers"][0]["wv"]
        x = O.dequantize(model["tok_embd"][1], model["tok_embd"][0][3], 64)
        xb = rms_norm(x, model["layers"][0]["attn_norm"], cfg.rms_eps)
        vrow = O.matmul(t, raw, 64, 64, xb[None], 1)[0]
        assert np.array_equal(o.caches[0][1][0, 0, 0], vrow.astype(np.float16))


# Inverse frequencies for head width 64 that the reference's own tests hold (values from Hugging
# Face Transformers' rope initializers; src/engine/ops.zig:292-343, compared there within 2e-6).
ROPE_PROBES = {
    "llama3": (dict(kind="llama3", factor=8.0, orig_ctx=8192, low_freq_factor=1.0, high_freq_factor=4.0), 500000.0,
               [(0, 1.0), (1, 6.636012793e-01), (7, 5.666961893e-02), (8, 3.760603070e-02), (12, 7.292665076e-03),
                (16, 5.248460220e-04), (20, 3.428102355e-05), (24, 6.647869668e-06), (31, 3.767322596e-07)]),
    "yarn": (dict(kind="yarn", factor=4.0, orig_ctx=4096), 10000.0,
             [(0, 1.0), (1, 7.498942018e-01), (7, 1.333521456e-01), (8, 1.000000015e-01), (12, 2.797399648e-02),
              (16, 6.538461894e-03), (20, 1.337886788e-03), (24, 2.500000119e-04), (31, 3.333803761e-05)]),
    "linear": (dict(kind="linear", factor=4.0), 10000.0,
               [(0, 0.25), (1, 1.874735504e-01), (16, 2.499999944e-03), (31, 3.333803761e-05)]),
}


@pytest.mark.parametrize("which", ["oracle", "host"])
@pytest.mark.parametrize("case", list(ROPE_PROBES))
def test_rope_inv_freq_reference_probes(which, case):
    """Both restatements of ropeInvFreq -- the oracle's and the host code that feeds the device pass
    (hk_amd/rope.py) -- against the reference's golden probes; plus the yarn magnitude
    (1.138629436 for factor 4), 1 for the others, and plain RoPE (no scaling: 1 and 4x the linear
    probe at 31), and frequency factors dividing the result."""
    from hk_amd.rope import RopeScaling, inv_freq, mscale
    from oracle.net_oracle import rope_inv_freq, rope_mscale

    kw, base, probes = ROPE_PROBES[case]
    sc = RopeScaling(**kw)
    f = rope_inv_freq if which == "oracle" else inv_freq
    ms = rope_mscale if which == "oracle" else mscale
    out = f(base, 64, sc)
    for i, want in probes:
        assert abs(float(out[i]) - want) <= 2e-6 * want, (case, i, float(out[i]), want)
    assert abs(ms(sc) - (1.138629436 if case == "yarn" else 1.0)) <= 1e-6
    plain = f(10000.0, 64, None)
    assert plain[0] == 1.0 and abs(float(plain[31]) - 4 * 3.333803761e-05) <= 1e-5 * 4 * 3.333803761e-05
    factors = 1.0 + np.arange(32, dtype=np.float32)
    with_f = f(10000.0, 64, None, factors)
    assert np.allclose(with_f, plain / factors, rtol=1e-6)
