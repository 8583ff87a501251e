"""The whole-network device pass (hkhip_net_* in include/hkhip.h), as hk's engine interface sees it
(reference src/backend/backend.zig:128-209 Device, src/cuda/engine.zig Engine): load the layers'
tensors (hk file-layout bytes, f32 vectors), run passes over the items of one or more sequences
(`forward_items`, each sequence in its own cache slot), read the logits of chosen items
(`logits_rows`), free a sequence's slot (`release`), run a partial network's leading layers on
hidden states the caller embedded (`forward_partial`), and size a network before creating it
(`bytes_needed`, `layer_bytes`: engine.zig:155-190)."""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import rope
from ._lib import NET_LAYER_FIELDS, Item, NetConfig, NetLayer, NetOptions, NetTensor, check, lib

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


@dataclass
class Options:
    """src/cuda/engine.zig:43-58 Options."""
    slots: int = 1
    layers: int = 0          # leading layers on the device; 0: all (fewer: a partial network)
    n_batch: int = 0         # most tokens per pass (0: buffers grown on demand)
    attn_merge_max: int = 0  # test knob: decode attention chunks merged inside the launch (0: 256)
    attn_gqa: int = 0        # decode attention kernel: 0 by size, 1 grouped (GQA, MFMA), 2 per head

    def c(self) -> NetOptions:
        return NetOptions(self.slots, self.layers, self.n_batch, self.attn_merge_max, self.attn_gqa)


# hkhip_item's layout (include/hkhip.h): u64 seq, u32 token, u32 pos -- 16 bytes, no padding.
_ITEM_DTYPE = np.dtype([("seq", "<u8"), ("token", "<u4"), ("pos", "<u4")])
assert _ITEM_DTYPE.itemsize == ctypes.sizeof(Item)


def _items(items) -> tuple:
    """(pointer, count, keep-alive array) of hkhip_item from (seq, token, pos) triples, built in
    bulk (a prompt's thousands of items)."""
    n = len(items)
    if n == 0:
        arr = np.zeros(1, _ITEM_DTYPE)
    elif isinstance(items, np.ndarray):  # an [n][3] array
        a = items.reshape(n, 3).astype(np.uint64)
        arr = np.empty(n, _ITEM_DTYPE)
        arr["seq"], arr["token"], arr["pos"] = a[:, 0], a[:, 1], a[:, 2]
    else:
        arr = np.fromiter((tuple(it) for it in items) if not isinstance(items[0], tuple) else items,
                          _ITEM_DTYPE, n)
    return arr.ctypes.data, n, arr


def _layer(tensors: dict, keep: list) -> NetLayer:
    return NetLayer(*[_tensor(tensors.get(n), keep) for n in NET_LAYER_FIELDS])


def bytes_needed(cfg: Config, model: dict, opts: Options | None = None) -> int:
    """hkhip_net_bytes_needed: device bytes (with the 64 MiB margin) a network of cfg / opts holds for
    the tensors of `model` (only their sizes and types are read)."""
    keep: list = []
    c, o = cfg.c(), (opts or Options()).c()
    layers = (NetLayer * cfg.n_layers)(*[_layer(l, keep) for l in model["layers"]])
    return int(lib().hkhip_net_bytes_needed(ctypes.byref(c), ctypes.byref(o), layers, _tensor(model["tok_embd"], keep),
                                            _tensor(model["out_norm"], keep), _tensor(model["output"], keep)))


def layer_bytes(cfg: Config, layer: dict) -> int:
    """hkhip_net_layer_bytes: device bytes of one layer's tensors."""
    keep: list = []
    c = cfg.c()
    return int(lib().hkhip_net_layer_bytes(ctypes.byref(c), ctypes.byref(_layer(layer, keep))))


class Net:
    def __init__(self, eng, cfg: Config, opts: Options | None = None):
        self.cfg = cfg
        self.eng = eng
        self.opts = opts or Options()
        self._h = ctypes.c_void_p()
        c, o = cfg.c(), self.opts.c()
        check(lib().hkhip_net_create_opts(eng._h, ctypes.byref(c), ctypes.byref(o), ctypes.byref(self._h)))

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
        check(lib().hkhip_net_load_layer(self._h, i, ctypes.byref(_layer(tensors, keep))))

    def load_io(self, tok_embd, out_norm, output) -> None:
        keep: list = []
        check(lib().hkhip_net_load_io(self._h, _tensor(tok_embd, keep), _tensor(out_norm, keep), _tensor(output, keep)))

    def load(self, model: dict) -> None:
        for i, layer in enumerate(model["layers"][:self.layer_count]):
            self.load_layer(i, layer)
        if not self.is_partial:
            self.load_io(model["tok_embd"], model["out_norm"], model["output"])

    # Device.forward / forwardPartial / logits / release / maxRows / layerCount / isPartial
    def forward_items(self, items) -> None:
        """One pass over (seq, token, pos) items of one or more sequences."""
        p, n, _keep = _items(items)
        check(lib().hkhip_net_forward_items(self._h, p, n))

    def forward_partial(self, items, hidden: np.ndarray) -> np.ndarray:
        """A partial network's pass: hidden [n][dim] in, the state after its last layer out."""
        p, n, _keep = _items(items)
        h = np.ascontiguousarray(hidden, dtype=np.float32).copy()
        assert h.shape == (n, self.cfg.dim)
        check(lib().hkhip_net_forward_partial(self._h, p, n, h.ctypes.data))
        return h

    def logits_rows(self, indices) -> np.ndarray:
        idx = np.ascontiguousarray(indices, dtype=np.uint32)
        out = np.empty((idx.size, self.cfg.vocab), np.float32)
        check(lib().hkhip_net_logits_rows(self._h, idx.ctypes.data, idx.size, out.ctypes.data))
        return out

    def logits_view(self, indices) -> np.ndarray:
        """The same rows as logits_rows, as the reference's Device.logits returns them
        (engine.zig:799-816): a view of the network's own (pinned) host buffer, valid until the
        next call on this network, no copy."""
        idx = np.ascontiguousarray(indices, dtype=np.uint32)
        p = ctypes.c_void_p()
        check(lib().hkhip_net_logits_view(self._h, idx.ctypes.data, idx.size, ctypes.byref(p)))
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_float)), shape=(idx.size, self.cfg.vocab))

    def release(self, seq: int) -> None:
        lib().hkhip_net_release(self._h, seq)

    @property
    def max_rows(self) -> int:
        return int(lib().hkhip_net_max_rows(self._h))

    @property
    def layer_count(self) -> int:
        return int(lib().hkhip_net_layer_count(self._h))

    @property
    def is_partial(self) -> bool:
        return bool(lib().hkhip_net_is_partial(self._h))

    def device_bytes(self) -> int:
        return int(lib().hkhip_net_device_bytes(self._h))

    # one sequence (seq 0), the last token's logits computed inside the pass
    def forward(self, tokens, pos0: int) -> None:
        toks = np.ascontiguousarray(tokens, dtype=np.uint32)
        check(lib().hkhip_net_forward(self._h, toks.ctypes.data, toks.size, pos0))

    def logits(self) -> np.ndarray:
        out = np.empty(self.cfg.vocab, np.float32)
        check(lib().hkhip_net_logits(self._h, out.ctypes.data))
        return out
