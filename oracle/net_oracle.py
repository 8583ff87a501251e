"""CPU restatement of hk's decoder forward pass (TEST INFRASTRUCTURE ONLY: tests/ use it as the
checker of the HIP network pass; the product never calls it).

Follows src/engine/cpu_backend.zig:237-331 (embed, forwardFrom, logitsFor) with the oracle's
restatement of the quantized products (oracle.matmul: quantizeA8 / quantizeQ8K of the input, then
hk's integer dots), src/engine/ops.zig rmsNorm (10-29), headNorm (31-38), ropeInvFreq without
scaling (96-146), ropeAngles (154-160), ropeApply (164-185), swiglu (70-80), and causal GQA
attention softmax(q k^T / sqrt(head_dim)) v over an f16 key/value cache (src/engine/kv.zig:1-11,
attention.zig:44-110), evaluated in float64 from the f16-rounded cache.
"""
from __future__ import annotations

import numpy as np

from . import oracle as O


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = x.astype(np.float32)
    ss = np.float32(np.sum(x.astype(np.float64) ** 2))
    inv = np.float32(1.0) / np.sqrt(ss / np.float32(x.size) + np.float32(eps))
    return (x * inv) * w


class Oracle:
    def __init__(self, cfg, model: dict):
        self.cfg, self.m = cfg, model
        hd, L = cfg.head_dim, cfg.n_layers
        self.kc = np.zeros((L, cfg.n_kv_heads, cfg.max_ctx, hd), np.float16)
        self.vc = np.zeros_like(self.kc)
        rd = cfg.rope_dim or hd
        self.inv_freq = np.array([np.float64(cfg.rope_base) ** (-2.0 * i / rd) for i in range(rd // 2)], np.float32)

    def _mm(self, mat, x, bias=None):
        raw, t = mat
        rows = raw.shape[0]
        return O.matmul(t, raw, rows, x.shape[1], x, x.shape[0], bias=bias, threads=8)

    def _rope(self, v: np.ndarray, pos: int) -> np.ndarray:
        c = self.cfg
        half = (c.rope_dim or c.head_dim) // 2
        ang = np.float32(pos) * self.inv_freq
        cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
        v = v.copy()
        if c.rope_neox:
            a, b = v[:half].copy(), v[half:2 * half].copy()
            v[:half], v[half:2 * half] = a * cs - b * sn, a * sn + b * cs
        else:
            a, b = v[0:2 * half:2].copy(), v[1:2 * half:2].copy()
            v[0:2 * half:2], v[1:2 * half:2] = a * cs - b * sn, a * sn + b * cs
        return v

    def forward(self, tokens, pos0: int) -> np.ndarray:
        """Runs tokens at positions pos0..; returns the last token's logits."""
        c, m = self.cfg, self.m
        n, hd = len(tokens), c.head_dim
        raw, t = m["tok_embd"]
        x = np.stack([O.dequantize(t, raw[tok], c.dim) for tok in tokens]).astype(np.float32)
        group = c.n_heads // c.n_kv_heads
        for li, L in enumerate(m["layers"]):
            xb = np.stack([rms_norm(x[i], L["attn_norm"], c.rms_eps) for i in range(n)])
            q = self._mm(L["wq"], xb, L.get("bq"))
            k = self._mm(L["wk"], xb, L.get("bk"))
            v = self._mm(L["wv"], xb, L.get("bv"))
            for i in range(n):
                pos = pos0 + i
                for h in range(c.n_heads):
                    s = q[i, h * hd:(h + 1) * hd]
                    if L.get("q_norm") is not None:
                        s = rms_norm(s, L["q_norm"], c.rms_eps)
                    q[i, h * hd:(h + 1) * hd] = self._rope(s, pos)
                for g in range(c.n_kv_heads):
                    s = k[i, g * hd:(g + 1) * hd]
                    if L.get("k_norm") is not None:
                        s = rms_norm(s, L["k_norm"], c.rms_eps)
                    self.kc[li, g, pos] = self._rope(s, pos).astype(np.float16)
                    self.vc[li, g, pos] = v[i, g * hd:(g + 1) * hd].astype(np.float16)
            att = np.zeros((n, c.n_heads * hd), np.float32)
            scale = 1.0 / np.sqrt(np.float64(hd))
            for i in range(n):
                pos = pos0 + i
                for h in range(c.n_heads):
                    g = h // group
                    kk = self.kc[li, g, :pos + 1].astype(np.float64)
                    vv = self.vc[li, g, :pos + 1].astype(np.float64)
                    sc = kk @ q[i, h * hd:(h + 1) * hd].astype(np.float64) * scale
                    p = np.exp(sc - sc.max())
                    att[i, h * hd:(h + 1) * hd] = (p @ vv) / p.sum()
            x = x + self._mm(L["wo"], att)
            xb = np.stack([rms_norm(x[i], L["ffn_norm"], c.rms_eps) for i in range(n)])
            gate = self._mm(L["w_gate"], xb)
            up = self._mm(L["w_up"], xb)
            with np.errstate(over="ignore"):
                hmid = (gate / (np.float32(1) + np.exp(-gate)) * up).astype(np.float32)
            x = x + self._mm(L["w_down"], hmid)
        xl = rms_norm(x[n - 1], m["out_norm"], c.rms_eps)
        return self._mm(m["output"], xl[None])[0]
