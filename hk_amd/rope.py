"""RoPE inverse frequencies and rotation magnitude, computed on the host as hk's model setup does
before it hands them to a device engine (reference src/engine/model.zig:123-124 calling
src/engine/ops.zig:93-152 ropeInvFreq / ropeMscale; scaling parameters and their defaults as in
src/engine/config.zig:48-62 RopeScaling). The HIP network pass takes both through
hkhip_net_config (inv_freq, rope_mscale), as hk's CUDA engine takes them at init."""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

KINDS = ("none", "linear", "llama3", "yarn")


@dataclass
class RopeScaling:
    kind: str = "none"
    factor: float = 1.0
    orig_ctx: int = 0              # context the model was trained with before scaling
    low_freq_factor: float = 1.0   # llama3 band
    high_freq_factor: float = 4.0
    beta_fast: float = 32.0        # yarn band (rotation counts)
    beta_slow: float = 1.0
    attn_factor: float = 1.0       # yarn magnitude multiplier

    def __post_init__(self):
        if self.kind not in KINDS:
            raise ValueError(f"rope scaling '{self.kind}' is not supported ({', '.join(KINDS)})")


def inv_freq(base: float, n_rot: int, r: RopeScaling | None = None, factors=None) -> np.ndarray:
    """n_rot / 2 inverse frequencies base^(-2i/n_rot), stretched by `r`, divided by the optional
    per-frequency factors (llama3 scaling as llama.cpp files carry it); float64 math, float32 out."""
    r = r or RopeScaling()
    half = n_rot // 2
    nr, b, f = float(n_rot), float(np.float32(base)), float(np.float32(r.factor))
    lo = hi = 0.0
    if r.kind == "yarn":
        ctx = float(r.orig_ctx)

        def corr(rot):
            return nr * math.log(ctx / (rot * 2.0 * math.pi)) / (2.0 * math.log(b))

        lo = max(0.0, math.floor(corr(float(np.float32(r.beta_fast)))))
        hi = min(nr - 1.0, math.ceil(corr(float(np.float32(r.beta_slow)))))
        if lo == hi:
            hi += 0.001
    out = np.empty(half, np.float32)
    for i in range(half):
        inv = b ** (-(2.0 * i) / nr)
        if r.kind == "linear":
            v = inv / f
        elif r.kind == "llama3":
            old = float(r.orig_ctx)
            lf, hf = float(np.float32(r.low_freq_factor)), float(np.float32(r.high_freq_factor))
            wavelen = 2.0 * math.pi / inv
            if wavelen < old / hf:
                v = inv
            elif wavelen > old / lf:
                v = inv / f
            else:
                smooth = (old / wavelen - lf) / (hf - lf)
                v = (1.0 - smooth) * inv / f + smooth * inv
        elif r.kind == "yarn":
            ramp = min(max((i - lo) / (hi - lo), 0.0), 1.0)
            keep = 1.0 - ramp
            v = (inv / f) * (1.0 - keep) + inv * keep
        else:
            v = inv
        if factors is not None:
            v /= float(np.float32(factors[i]))
        out[i] = np.float32(v)
    return out


def mscale(r: RopeScaling | None) -> float:
    """The multiplier of every cos and sin: attn_factor * (1 + 0.1 ln(factor)) for yarn, else 1."""
    if r is None or r.kind != "yarn":
        return 1.0
    return float(np.float32(r.attn_factor) * np.float32(1.0 + 0.1 * math.log(float(np.float32(r.factor)))))
