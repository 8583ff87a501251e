"""CPU restatement of hk's decoder forward pass (TEST INFRASTRUCTURE ONLY: tests/ use it as the
checker of the HIP network pass; the product never calls it).

Follows src/engine/cpu_backend.zig:237-331 (embed, forwardFrom, logitsFor) with the oracle's
restatement of the quantized products (oracle.matmul: quantizeA8 / quantizeQ8K of the input, then
hk's integer dots), src/engine/ops.zig rmsNorm (10-29), headNorm (31-38), ropeInvFreq with the
none / linear / llama3 / yarn scalings and frequency factors (93-146), ropeMscale (148-152),
ropeAngles (154-160), ropeApply (164-185), swiglu (70-80), and causal GQA
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


def rope_inv_freq(base, n_rot: int, sc=None, factors=None) -> np.ndarray:
    """src/engine/ops.zig:96-146 ropeInvFreq: base^(-2i/n_rot) in float64, stretched by the scaling
    `sc` (fields of src/engine/config.zig:48-62; None: no scaling), divided by the optional
    per-frequency factors, rounded to float32."""
    i = np.arange(n_rot // 2, dtype=np.float64)
    nr, b = np.float64(n_rot), np.float64(np.float32(base))
    inv = b ** (-(2.0 * i) / nr)
    kind = getattr(sc, "kind", "none")
    if kind != "none":
        f = np.float64(np.float32(sc.factor))
    if kind == "linear":
        inv = inv / f
    elif kind == "llama3":
        old = np.float64(sc.orig_ctx)
        lf, hf = np.float64(np.float32(sc.low_freq_factor)), np.float64(np.float32(sc.high_freq_factor))
        wl = 2.0 * np.pi / inv
        smooth = (old / wl - lf) / (hf - lf)
        mid = (1.0 - smooth) * inv / f + smooth * inv
        inv = np.where(wl < old / hf, inv, np.where(wl > old / lf, inv / f, mid))
    elif kind == "yarn":
        ctx = np.float64(sc.orig_ctx)
        dim = lambda rot: nr * np.log(ctx / (rot * 2.0 * np.pi)) / (2.0 * np.log(b))
        lo = max(0.0, np.floor(dim(np.float64(np.float32(sc.beta_fast)))))
        hi = min(nr - 1.0, np.ceil(dim(np.float64(np.float32(sc.beta_slow)))))
        if lo == hi:
            hi += 0.001
        ramp = np.clip((i - lo) / (hi - lo), 0.0, 1.0)
        inv = (inv / f) * ramp + inv * (1.0 - ramp)
    if factors is not None:
        inv = inv / np.asarray(factors, np.float32).astype(np.float64)
    return inv.astype(np.float32)


def rope_mscale(sc=None) -> float:
    """src/engine/ops.zig:148-152 ropeMscale: attn_factor * (0.1 ln(factor) + 1) for yarn, else 1."""
    if getattr(sc, "kind", "none") != "yarn":
        return 1.0
    return float(np.float32(sc.attn_factor) * np.float32(1.0 + 0.1 * np.log(np.float64(np.float32(sc.factor)))))


class Oracle:
    """hk's CPU forward over items of one or more sequences, each with its own f16 cache (a
    KvCache per sequence, src/engine/kv.zig:22-29). `forward_items` mirrors Device.forward /
    forwardPartial (src/backend/backend.zig:158-177): every layer writes the keys and values of all
    items before any attends (src/cuda/engine.zig:674-675: "a token sees its predecessors in the
    same pass"), an item attends to positions 0..pos of its own sequence; `logits_rows` mirrors
    Device.logits (backend.zig:189-194) / logitsFor (cpu_backend.zig:324-331)."""

    def __init__(self, cfg, model: dict):
        self.cfg, self.m = cfg, model
        self.caches: dict = {}  # seq -> (keys, values) [layer][kv head][max_ctx][hd] f16
        rd = cfg.rope_dim or cfg.head_dim
        sc = getattr(cfg, "rope_scaling", None)
        self.inv_freq = rope_inv_freq(cfg.rope_base, rd, sc, getattr(cfg, "rope_freq_factors", None))
        self.mscale = rope_mscale(sc)
        self.hidden = None

    def _cache(self, seq):
        if seq not in self.caches:
            c = self.cfg
            kc = np.zeros((c.n_layers, c.n_kv_heads, c.max_ctx, c.head_dim), np.float16)
            self.caches[seq] = (kc, np.zeros_like(kc))
        return self.caches[seq]

    def release(self, seq) -> None:
        self.caches.pop(seq, None)

    def _mm(self, mat, x, bias=None):
        raw, t = mat
        rows = raw.shape[0]
        return O.matmul(t, raw, rows, x.shape[1], x, x.shape[0], bias=bias, threads=8)

    def _rope(self, v: np.ndarray, pos: int) -> np.ndarray:
        c = self.cfg
        half = (c.rope_dim or c.head_dim) // 2
        ang = np.float32(pos) * self.inv_freq
        cs = (np.cos(ang).astype(np.float32) * np.float32(self.mscale)).astype(np.float32)
        sn = (np.sin(ang).astype(np.float32) * np.float32(self.mscale)).astype(np.float32)
        v = v.copy()
        if c.rope_neox:
            a, b = v[:half].copy(), v[half:2 * half].copy()
            v[:half], v[half:2 * half] = a * cs - b * sn, a * sn + b * cs
        else:
            a, b = v[0:2 * half:2].copy(), v[1:2 * half:2].copy()
            v[0:2 * half:2], v[1:2 * half:2] = a * cs - b * sn, a * sn + b * cs
        return v

    def embed(self, tokens) -> np.ndarray:
        c = self.cfg
        raw, t = self.m["tok_embd"]
        return np.stack([O.dequantize(t, raw[tok], c.dim) for tok in tokens]).astype(np.float32)

    def forward_items(self, items, hidden: np.ndarray | None = None, layers: int | None = None,
                      first: int = 0) -> np.ndarray:
        """Runs (seq, token, pos) items through layers [first, layers) (all by default), from their
        embeddings or from `hidden` [n][dim]; returns the hidden states after the last layer run
        (a partial device's leading layers, then the CPU's rest: cpu_backend.zig forwardFrom)."""
        c, m = self.cfg, self.m
        n, hd = len(items), c.head_dim
        x = self.embed([t for _, t, _ in items]) if hidden is None else np.array(hidden, np.float32)
        group = c.n_heads // c.n_kv_heads
        nl = c.n_layers if layers is None else layers
        for li in range(first, nl):
            L = m["layers"][li]
            xb = np.stack([rms_norm(x[i], L["attn_norm"], c.rms_eps) for i in range(n)])
            q = self._mm(L["wq"], xb, L.get("bq"))
            k = self._mm(L["wk"], xb, L.get("bk"))
            v = self._mm(L["wv"], xb, L.get("bv"))
            for i, (seq, _, pos) in enumerate(items):
                kc, vc = self._cache(seq)
                for h in range(c.n_heads):
                    s = q[i, h * hd:(h + 1) * hd]
                    if L.get("q_norm") is not None:
                        s = rms_norm(s, L["q_norm"], c.rms_eps)
                    q[i, h * hd:(h + 1) * hd] = self._rope(s, pos)
                for g in range(c.n_kv_heads):
                    s = k[i, g * hd:(g + 1) * hd]
                    if L.get("k_norm") is not None:
                        s = rms_norm(s, L["k_norm"], c.rms_eps)
                    kc[li, g, pos] = self._rope(s, pos).astype(np.float16)
                    vc[li, g, pos] = v[i, g * hd:(g + 1) * hd].astype(np.float16)
            att = np.zeros((n, c.n_heads * hd), np.float32)
            scale = 1.0 / np.sqrt(np.float64(hd))
            for i, (seq, _, pos) in enumerate(items):
                kc, vc = self._cache(seq)
                for h in range(c.n_heads):
                    g = h // group
                    kk = kc[li, g, :pos + 1].astype(np.float64)
                    vv = vc[li, g, :pos + 1].astype(np.float64)
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
        self.hidden = x
        return x

    def logits_rows(self, indices) -> np.ndarray:
        """Logits of the given items of the last forward_items, one row each."""
        m, c = self.m, self.cfg
        xl = np.stack([rms_norm(self.hidden[i], m["out_norm"], c.rms_eps) for i in indices])
        return self._mm(m["output"], xl)

    def forward(self, tokens, pos0: int) -> np.ndarray:
        """Runs tokens of sequence 0 at positions pos0..; returns the last token's logits."""
        self.forward_items([(0, int(t), pos0 + i) for i, t in enumerate(tokens)])
        return self.logits_rows([len(tokens) - 1])[0]
