"""The whole-network device pass (hkhip_net_* in include/hkhip.h), as hk's engine interface sees it:
load the layers' tensors (hk file-layout bytes, f32 vectors), run forward passes over one
sequence, read the last token's logits (reference src/cuda/engine.zig:646-797, src/backend/backend.zig
Device.forward / logits)."""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import rope
from ._lib import NET_LAYER_FIELDS, NetConfig, NetLayer, NetTensor, check, lib

F32 = 0x00  # hk StorageType f32


@dataclass
class Config:
    dim: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn_dim: int
    vocab: int
    max_ctx: int
    rope_dim: int = 0          # 0: head_dim
    rope_neox: bool = True     # pairs (i, i + half); False: (2i, 2i + 1)
    rms_eps: float = 1e-6
    rope_base: float = 1e6
    rope_scaling: rope.RopeScaling | None = None  # none / linear / llama3 / yarn
    rope_freq_factors: np.ndarray | None = None   # per-frequency divisors (a file's rope_freqs.weight)

    def inv_freq(self) -> np.ndarray:
        return rope.inv_freq(self.rope_base, self.rope_dim or self.head_dim, self.rope_scaling, self.rope_freq_factors)

    def c(self) -> NetConfig:
        self._inv = np.ascontiguousarray(self.inv_freq(), np.float32)  # read by hkhip_net_create
        return NetConfig(self.dim, self.n_layers, self.n_heads, self.n_kv_heads, self.head_dim, self.ffn_dim,
                         self.vocab, self.rope_dim or self.head_dim, int(self.rope_neox), self.max_ctx,
                         self.rms_eps, self.rope_base, self._inv.ctypes.data, rope.mscale(self.rope_scaling))


def _tensor(v, keep: list) -> NetTensor:
    """(raw uint8 blocks, type) for a matrix, a float32 array for a vector, None when absent."""
    if v is None:
        return NetTensor(None, 0, 0)
    if isinstance(v, tuple):
        raw, t = v
        raw = np.ascontiguousarray(raw).view(np.uint8)
    else:
        raw, t = np.ascontiguousarray(v, dtype=np.float32), F32
    keep.append(raw)
    return NetTensor(raw.ctypes.data, raw.nbytes, t)


class Net:
    def __init__(self, eng, cfg: Config):
        self.cfg = cfg
        self.eng = eng
        self._h = ctypes.c_void_p()
        c = cfg.c()
        check(lib().hkhip_net_create(eng._h, ctypes.byref(c), ctypes.byref(self._h)))

    def close(self) -> None:
        if self._h:
            lib().hkhip_net_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def load_layer(self, i: int, tensors: dict) -> None:
        keep: list = []
        layer = NetLayer(*[_tensor(tensors.get(n), keep) for n in NET_LAYER_FIELDS])
        check(lib().hkhip_net_load_layer(self._h, i, ctypes.byref(layer)))

    def load_io(self, tok_embd, out_norm, output) -> None:
        keep: list = []
        check(lib().hkhip_net_load_io(self._h, _tensor(tok_embd, keep), _tensor(out_norm, keep), _tensor(output, keep)))

    def load(self, model: dict) -> None:
        for i, layer in enumerate(model["layers"]):
            self.load_layer(i, layer)
        self.load_io(model["tok_embd"], model["out_norm"], model["output"])

    def forward(self, tokens, pos0: int) -> None:
        toks = np.ascontiguousarray(tokens, dtype=np.uint32)
        check(lib().hkhip_net_forward(self._h, toks.ctypes.data, toks.size, pos0))

    def logits(self) -> np.ndarray:
        out = np.empty(self.cfg.vocab, np.float32)
        check(lib().hkhip_net_logits(self._h, out.ctypes.data))
        return out
