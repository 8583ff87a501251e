"""Synthetic weights and activations of the shapes the benchmarks and tests use.

Blocks are random but valid: quant bytes are uniform; scale fields are finite f16 drawn as
|N(0, 0.02)| magnitudes (the spread of trained weights' block scales) (per format below); activations are N(0, 1) f32, with an
optional fraction of outliers at +-20. The same generator runs on NumPy (host, tests and the
CPU baseline) or torch (device, for multi-GB benchmark matrices).

  Q8_0   qs uniform in [-127, 127];           d = |N(0,0.02)| / 127 * 4
  Q4_K   qs and the 12 scale bytes uniform;   d = dmin = |N(0,0.02)| / 63
  Q6_K   ql / qh uniform, scales in [-32,31]; d = |N(0,0.02)| / 127
  IQ4_NL indices uniform;                     d = |N(0,0.02)|
  Q4_0 / Q5_0  quants uniform;                d = |N(0,0.02)| / 8 (/ 16)
  Q4_1 / Q5_1  quants uniform;                d = |N(0,0.02)| / 16 (/ 32), m = -|N(0,0.02)|
  Q5_K   as Q4_K (qh uniform);                d = dmin = |N(0,0.02)| / 63
  IQ4_XS indices and scale bits uniform;      d = |N(0,0.02)| / 1024
"""
from __future__ import annotations

import numpy as np

from . import formats

SEED_BASE = 20261201


def seed_for(config: int, tensor: int) -> int:
    """seed = 20261201 + config * 1000 + tensor index."""
    return SEED_BASE + config * 1000 + tensor


def _f16_scales_np(rng, nb: int, div: float) -> np.ndarray:
    return (np.abs(rng.normal(0.0, 0.02, nb)) / div).astype(np.float16)


def weights_np(t: int, rows: int, cols: int, seed: int) -> np.ndarray:
    """Random valid blocks in hk's file layout, as a [rows, row_bytes] uint8 array."""
    elems, bb = formats.INFO[t]
    nb = rows * (cols // elems)
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    if t == formats.Q8_0:
        raw[:, 2:34] = rng.integers(-127, 128, size=(nb, 32)).astype(np.int8).view(np.uint8)
        raw[:, 0:2] = _f16_scales_np(rng, nb, 127.0 / 4.0).view(np.uint8).reshape(nb, 2)
    elif t in (formats.Q4_K, formats.Q5_K):
        raw[:, 0:2] = _f16_scales_np(rng, nb, 63.0).view(np.uint8).reshape(nb, 2)
        raw[:, 2:4] = _f16_scales_np(rng, nb, 63.0).view(np.uint8).reshape(nb, 2)
    elif t == formats.IQ4_XS:
        raw[:, 0:2] = _f16_scales_np(rng, nb, 1024.0).view(np.uint8).reshape(nb, 2)
    elif t == formats.Q6_K:
        raw[:, 192:208] = rng.integers(-32, 32, size=(nb, 16)).astype(np.int8).view(np.uint8)
        raw[:, 208:210] = _f16_scales_np(rng, nb, 127.0).view(np.uint8).reshape(nb, 2)
    elif t == formats.IQ4_NL:
        raw[:, 0:2] = _f16_scales_np(rng, nb, 1.0).view(np.uint8).reshape(nb, 2)
    elif t in _FB_D:
        for off, div in _FB_D[t]:
            raw[:, off:off + 2] = _f16_scales_np(rng, nb, div).view(np.uint8).reshape(nb, 2)
    elif t == formats.IQ1_M:
        # the f16 scale is the top nibbles of the four 16-bit scale words (bytes 48..55)
        bits = _f16_scales_np(rng, nb, 1.0).view(np.uint16).astype(np.uint32)
        for i in range(4):
            hi = (bits >> (4 * i)) & 0xF
            raw[:, 49 + 2 * i] = (raw[:, 49 + 2 * i] & 0x0F) | (hi << 4).astype(np.uint8)
    elif t == formats.MXFP4:
        raw[:, 0] = rng.integers(118, 126, size=nb)  # E8M0 exponents around 2^-4 .. 2^-9
    elif t in _LOW_BIT:
        div, has_m = _LOW_BIT[t]
        raw[:, 0:2] = _f16_scales_np(rng, nb, div).view(np.uint8).reshape(nb, 2)
        if has_m:
            raw[:, 2:4] = (-_f16_scales_np(rng, nb, 1.0)).view(np.uint8).reshape(nb, 2)
    return raw.reshape(rows, -1)


# The float-decode formats' f16 scale fields: (byte offset, divisor of |N(0, 0.02)|).
_FB_D = {formats.Q2_K: ((80, 1.0), (82, 1.0)), formats.Q3_K: ((108, 1.0),), formats.IQ2_XXS: ((0, 1.0),),
         formats.IQ2_XS: ((0, 1.0),), formats.IQ2_S: ((0, 1.0),), formats.IQ3_XXS: ((0, 1.0),),
         formats.IQ3_S: ((0, 1.0),), formats.IQ1_S: ((0, 1.0),), formats.TQ1_0: ((52, 1.0),),
         formats.TQ2_0: ((64, 1.0),)}

# Q4_0 / Q4_1 / Q5_0 / Q5_1: scale divisor, has an offset m (f16 at bytes 2..3).
_LOW_BIT = {formats.Q4_0: (8.0, False), formats.Q4_1: (16.0, True), formats.Q5_0: (16.0, False),
            formats.Q5_1: (32.0, True)}


def activations_np(n: int, k: int, seed: int, outliers: float = 0.0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    x = rng.normal(0.0, 1.0, size=(n, k)).astype(np.float32)
    if outliers > 0:
        mask = rng.random((n, k)) < outliers
        x[mask] = np.where(rng.random(int(mask.sum())) < 0.5, -20.0, 20.0).astype(np.float32)
    return x


def weights_torch(t: int, rows: int, cols: int, seed: int, device="cuda"):
    """Same distribution as weights_np, generated on the device (for multi-GB matrices)."""
    import torch

    elems, bb = formats.INFO[t]
    nb = rows * (cols // elems)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    raw = torch.randint(0, 256, (nb, bb), dtype=torch.uint8, device=device, generator=g)

    def scales(div):
        return (torch.randn(nb, device=device, generator=g) * 0.02).abs().div_(div).half().view(torch.uint8).view(nb, 2)

    if t == formats.Q8_0:
        raw[:, 2:34] = torch.randint(-127, 128, (nb, 32), device=device, generator=g).to(torch.int8).view(torch.uint8)
        raw[:, 0:2] = scales(127.0 / 4.0)
    elif t in (formats.Q4_K, formats.Q5_K):
        raw[:, 0:2] = scales(63.0)
        raw[:, 2:4] = scales(63.0)
    elif t == formats.IQ4_XS:
        raw[:, 0:2] = scales(1024.0)
    elif t == formats.Q6_K:
        raw[:, 192:208] = torch.randint(-32, 32, (nb, 16), device=device, generator=g).to(torch.int8).view(torch.uint8)
        raw[:, 208:210] = scales(127.0)
    elif t == formats.IQ4_NL:
        raw[:, 0:2] = scales(1.0)
    elif t in _LOW_BIT:
        div, has_m = _LOW_BIT[t]
        raw[:, 0:2] = scales(div)
        if has_m:
            raw[:, 2:4] = (-(torch.randn(nb, device=device, generator=g) * 0.02).abs()).half().view(torch.uint8).view(nb, 2)
    return raw.view(rows, -1)


def model_np(cfg, fmt: int, seed: int, out_fmt: int | None = None, embd_fmt: int | None = None,
             qk_norm: bool = True, bias: bool = False) -> dict:
    """A random decoder of `cfg`'s shape (hk_amd.net.Config): matrices in `fmt` (output in out_fmt,
    embedding in embd_fmt) as (raw blocks, type); norms 1 + N(0, 0.1); optional q/k norms and
    q/k/v biases. Same dict layout as hk_amd.net.Net.load takes."""
    rng = np.random.default_rng(seed)
    qd, kvd = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim

    def vec(n, base=1.0, sd=0.1):
        return (base + sd * rng.standard_normal(n)).astype(np.float32)

    def mat(t, rows, cols):
        return weights_np(t, rows, cols, int(rng.integers(1 << 30))), t

    layers = []
    for _ in range(cfg.n_layers):
        layers.append({
            "attn_norm": vec(cfg.dim), "ffn_norm": vec(cfg.dim),
            "wq": mat(fmt, qd, cfg.dim), "wk": mat(fmt, kvd, cfg.dim), "wv": mat(fmt, kvd, cfg.dim),
            "wo": mat(fmt, cfg.dim, qd), "w_gate": mat(fmt, cfg.ffn_dim, cfg.dim), "w_up": mat(fmt, cfg.ffn_dim, cfg.dim),
            "w_down": mat(fmt, cfg.dim, cfg.ffn_dim),
            "q_norm": vec(cfg.head_dim) if qk_norm else None, "k_norm": vec(cfg.head_dim) if qk_norm else None,
            "bq": vec(qd, 0.0, 0.5) if bias else None, "bk": vec(kvd, 0.0, 0.5) if bias else None,
            "bv": vec(kvd, 0.0, 0.5) if bias else None,
        })
    return {"layers": layers, "tok_embd": mat(embd_fmt or fmt, cfg.vocab, cfg.dim), "out_norm": vec(cfg.dim),
            "output": mat(out_fmt or fmt, cfg.vocab, cfg.dim)}
