"""hk's .hk model container, read-only and zero-copy: the file is memory-mapped, tensors are
views of the mapping (hk's weights.Mat, reference src/engine/weights.zig:1-34), and a decoder's
tensors upload straight from those views into the HIP network pass (hk_amd.net).

Layouts followed (reference files):
  FileHeader, 128 bytes, little endian          src/format.zig:133-163
  metadata: key u16 + bytes, tag u8, len u32, value   src/metadata.zig:225-300
  tensor table: name u16 + bytes, type, tile layout, sparsity, ndim u8, shape u64 x ndim,
    data / residual / scale offset + size u64 x 6, block_size u16, sparsity_ratio f32
                                                src/tensor_toc.zig:39-101
  header / range validation                     src/reader.zig:20-60
  configuration from metadata                   src/engine/config.zig:225-320 fromMetadata,
                                                163-223 parseRopeScaling
  tensor names, shapes, tied output              src/engine/weights.zig:96-240
"""
from __future__ import annotations

import struct
from dataclasses import dataclass

import numpy as np

from . import formats

MAGIC = b"HKNT"
VERSION_MAJOR = 1
HEADER = struct.Struct("<4sHHIHHQQQQQQQQQH38s")  # format.zig:133-152 FileHeader
assert HEADER.size == 128

# metadata value tags (format.zig MetadataValueType)
VAL_STRING, VAL_INT64, VAL_FLOAT64, VAL_BOOL, VAL_JSON, VAL_BYTES = 1, 2, 3, 4, 5, 6
F32, F16, BF16 = 0x00, 0x01, 0x02


class HkFormatError(ValueError):
    pass


@dataclass
class Entry:
    """One tensor table entry (format.zig TensorEntry)."""
    name: str
    t: int
    tile_layout: int
    sparsity: int
    shape: tuple
    data_offset: int
    data_size: int
    residual_offset: int = 0
    residual_size: int = 0
    scale_offset: int = 0
    scale_size: int = 0
    block_size: int = 32
    sparsity_ratio: float = 0.0


class _Reader:
    def __init__(self, buf, what: str):
        self.b, self.p, self.what = buf, 0, what

    def take(self, n: int) -> bytes:
        if self.p + n > len(self.b):
            raise HkFormatError(f"{self.what} is truncated")
        out = bytes(self.b[self.p:self.p + n])
        self.p += n
        return out

    def u(self, fmt: str):
        s = struct.calcsize(fmt)
        return struct.unpack(fmt, self.take(s))[0]


def _end(off: int, size: int, total: int, what: str) -> int:
    if off + size > total or off + size < off:
        raise HkFormatError(f"{what} [{off}, {off + size}) lies outside the {total}-byte file")
    return off + size


class HkFile:
    """A memory-mapped .hk container: header, metadata, tensor table (reader.zig HKReader.open)."""

    def __init__(self, path: str):
        self.path = path
        self.map = np.memmap(path, dtype=np.uint8, mode="r")
        n = self.map.size
        if n < HEADER.size:
            raise HkFormatError("file too small for the 128-byte header")
        h = HEADER.unpack(bytes(self.map[:HEADER.size]))
        (magic, vmaj, vmin, self.flags, self.alignment, self.split_index, self.tensor_count, self.kv_count,
         meta_off, meta_size, toc_off, toc_size, self.data_offset, self.appendix_offset, self.checksum,
         self.split_count, _) = h
        if magic != MAGIC or vmaj != VERSION_MAJOR:
            raise HkFormatError(f"not an hk v{VERSION_MAJOR} container (magic {magic!r}, version {vmaj}.{vmin})")
        self.version = (vmaj, vmin)
        self.metadata = self._metadata(self.map[meta_off:_end(meta_off, meta_size, n, "metadata")])
        self.entries = self._toc(self.map[toc_off:_end(toc_off, toc_size, n, "tensor table")])
        self.by_name = {e.name: e for e in self.entries}
        for e in self.entries:
            _end(e.data_offset, e.data_size, n, f"tensor '{e.name}'")

    def _metadata(self, buf) -> dict:
        r, out = _Reader(buf, "metadata"), {}
        for _ in range(self.kv_count):
            key = r.take(r.u("<H")).decode()
            tag, vlen = r.u("<B"), r.u("<I")
            raw = r.take(vlen)
            if tag in (VAL_STRING, VAL_JSON):
                out[key] = raw.decode()
            elif tag == VAL_INT64:
                out[key] = struct.unpack("<q", raw)[0]
            elif tag == VAL_FLOAT64:
                out[key] = struct.unpack("<d", raw)[0]
            elif tag == VAL_BOOL:
                out[key] = bool(raw[0]) if raw else False
            else:
                out[key] = raw
        return out

    def _toc(self, buf) -> list:
        r, out = _Reader(buf, "tensor table"), []
        for _ in range(self.tensor_count):
            name = r.take(r.u("<H")).decode()
            t, layout, sparsity, ndim = r.u("<B"), r.u("<B"), r.u("<B"), r.u("<B")
            if ndim > 8:
                raise HkFormatError(f"tensor '{name}' has {ndim} dimensions (at most 8)")
            shape = tuple(r.u("<Q") for _ in range(ndim))
            vals = [r.u("<Q") for _ in range(6)]
            block, ratio = r.u("<H"), r.u("<f")
            out.append(Entry(name, t, layout, sparsity, shape, *vals, block, ratio))
        return out

    def close(self) -> None:
        self.map = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- tensors -------------------------------------------------------------------------------
    def data(self, name: str) -> np.ndarray:
        """The tensor's bytes: a view of the mapping, no copy (reader.zig getTensorData)."""
        e = self.entry(name)
        return self.map[e.data_offset:e.data_offset + e.data_size]

    def entry(self, name: str) -> Entry:
        try:
            return self.by_name[name]
        except KeyError:
            raise HkFormatError(f"tensor '{name}' not found") from None

    def mat(self, name: str, rows: int, cols: int):
        """(bytes view, type) of a [rows, cols] matrix, checked as weights.zig mat() checks it."""
        e = self.entry(name)
        if len(e.shape) != 2 or e.shape != (rows, cols):
            raise HkFormatError(f"tensor '{name}' has shape {list(e.shape)}, expected [{rows}, {cols}]")
        if e.t not in formats.INFO:
            raise HkFormatError(f"tensor '{name}' uses storage type 0x{e.t:02x}, which this build cannot run")
        want = formats.matrix_bytes(e.t, rows, cols)
        if e.data_size != want:
            raise HkFormatError(f"tensor '{name}' holds {e.data_size} bytes, [{rows}, {cols}] needs {want}")
        return self.data(name).reshape(rows, -1), e.t

    def vec(self, name: str, n: int) -> np.ndarray:
        """An f32 vector (weights.zig vec(): f32 as stored, f16 / bf16 converted)."""
        e = self.entry(name)
        if int(np.prod(e.shape)) != n:
            raise HkFormatError(f"tensor '{name}' has {int(np.prod(e.shape))} elements, expected {n}")
        raw = self.data(name)
        if e.t == F32 and e.data_size == 4 * n:
            return np.frombuffer(raw, "<f4").copy()
        if e.t == F16 and e.data_size == 2 * n:
            return np.frombuffer(raw, "<f2").astype(np.float32)
        if e.t == BF16 and e.data_size == 2 * n:
            return (np.frombuffer(raw, "<u2").astype(np.uint32) << 16).view(np.float32)
        raise HkFormatError(f"vector tensor '{name}' must be f32, f16 or bf16 of {n} values")

    # -- the decoder -----------------------------------------------------------------------
    def config(self, max_ctx: int):
        """hk_amd.net.Config from the metadata (config.zig:225-320 fromMetadata)."""
        from .net import Config

        m = self.metadata
        arch = m.get("general.architecture")
        if arch is None:
            raise HkFormatError("model metadata has no 'general.architecture'")
        fam = {"llama": "llama", "mistral": "llama", "qwen2": "qwen2", "qwen3": "qwen3"}.get(arch)
        if fam is None:
            raise HkFormatError(f"architecture '{arch}' is not supported (llama, mistral, qwen2, qwen3)")

        def need(k):
            if f"{arch}.{k}" not in m:
                raise HkFormatError(f"missing '{arch}.{k}'")
            return int(m[f"{arch}.{k}"])

        def opt(k, d):
            return m.get(f"{arch}.{k}", d)

        dim, n_heads = need("embedding_length"), need("attention.head_count")
        n_kv = int(opt("attention.head_count_kv", n_heads))
        if n_heads % n_kv:
            raise HkFormatError(f"head_count {n_heads} is not a multiple of head_count_kv {n_kv}")
        head_dim = int(opt("attention.key_length", 0)) or dim // n_heads
        # A sliding window changes which positions are visible: refused, as config.zig:271-279 does.
        if int(opt("attention.sliding_window", 0) or 0) > 0:
            raise HkFormatError(f"sliding window attention ({int(opt('attention.sliding_window', 0))}) is not supported")
        rope_dim = int(opt("rope.dimension_count", head_dim))
        scaling = self._rope_scaling(arch, int(opt("context_length", 2048)), rope_dim)
        factors = None
        if "rope_freqs.weight" in self.by_name:  # llama3 scaling as llama.cpp files carry it
            factors = self.vec("rope_freqs.weight", rope_dim // 2)
            if not (np.isfinite(factors).all() and (factors > 0).all()):
                raise HkFormatError("'rope_freqs.weight' holds a value that is not a positive number")
        style = m.get("hk.rope_style", "norm" if fam == "llama" else "neox")
        vocab = self.entry("token_embd.weight").shape[0]
        cfg = Config(dim=dim, n_layers=need("block_count"), n_heads=n_heads, n_kv_heads=n_kv, head_dim=head_dim,
                     ffn_dim=need("feed_forward_length"), vocab=vocab, max_ctx=max_ctx, rope_dim=rope_dim,
                     rope_neox=style == "neox", rms_eps=float(opt("attention.layer_norm_rms_epsilon", 1e-5)),
                     rope_base=float(opt("rope.freq_base", 10000.0)), rope_scaling=scaling, rope_freq_factors=factors)
        cfg.qk_norm, cfg.qkv_bias = fam == "qwen3", fam == "qwen2"
        return cfg

    def _rope_scaling(self, arch: str, ctx_train: int, rope_dim: int):
        """RopeScaling from the metadata (config.zig:163-223 parseRopeScaling): the type, or a bare
        factor meaning linear; factor >= 1; the original context (default the training context);
        llama3's band (hk.rope.low/high_freq_factor), yarn's (hk.rope.beta_fast/slow) and magnitude."""
        from .rope import KINDS, RopeScaling

        m = self.metadata
        kind = m.get(f"{arch}.rope.scaling.type")
        factor = m.get(f"{arch}.rope.scaling.factor")
        if kind is None:
            kind = "linear" if factor is not None else "none"
        if kind not in KINDS:
            raise HkFormatError(f"rope scaling type '{kind}' is not supported (supported: {', '.join(KINDS)})")
        if kind == "none":
            return None
        if factor is None:
            raise HkFormatError(f"rope scaling '{kind}' needs '{arch}.rope.scaling.factor'")
        factor = float(factor)
        if not (np.isfinite(factor) and factor >= 1.0):
            raise HkFormatError(f"rope scaling factor {factor} must be at least 1")
        r = RopeScaling(kind, factor, int(m.get(f"{arch}.rope.scaling.original_context_length", ctx_train)))
        if kind == "llama3":
            r.low_freq_factor = float(m.get("hk.rope.low_freq_factor", r.low_freq_factor))
            r.high_freq_factor = float(m.get("hk.rope.high_freq_factor", r.high_freq_factor))
            if not (0 < r.low_freq_factor < r.high_freq_factor):
                raise HkFormatError("llama3 rope scaling needs 0 < low_freq_factor < high_freq_factor")
        elif kind == "yarn":
            r.beta_fast = float(m.get("hk.rope.beta_fast", r.beta_fast))
            r.beta_slow = float(m.get("hk.rope.beta_slow", r.beta_slow))
            r.attn_factor = float(m.get(f"{arch}.rope.scaling.attn_factor", r.attn_factor))
            if not (r.beta_fast > 0 and r.beta_slow > 0 and r.attn_factor > 0):
                raise HkFormatError("yarn rope scaling needs positive beta_fast, beta_slow and attn_factor")
        if kind != "linear" and (r.orig_ctx == 0 or rope_dim == 0):
            raise HkFormatError("rope scaling needs the original context length")
        return r

    def model(self, cfg) -> dict:
        """The decoder's tensors (weights.zig:96-176): matrices as views of the mapping, vectors f32;
        the output projection falls back to the embedding when the file ties them."""
        qd, kvd = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
        layers = []
        for i in range(cfg.n_layers):
            b = f"blk.{i}."
            L = {"attn_norm": self.vec(b + "attn_norm.weight", cfg.dim),
                 "wq": self.mat(b + "attn_q.weight", qd, cfg.dim), "wk": self.mat(b + "attn_k.weight", kvd, cfg.dim),
                 "wv": self.mat(b + "attn_v.weight", kvd, cfg.dim), "wo": self.mat(b + "attn_output.weight", cfg.dim, qd),
                 "ffn_norm": self.vec(b + "ffn_norm.weight", cfg.dim),
                 "w_gate": self.mat(b + "ffn_gate.weight", cfg.ffn_dim, cfg.dim),
                 "w_up": self.mat(b + "ffn_up.weight", cfg.ffn_dim, cfg.dim),
                 "w_down": self.mat(b + "ffn_down.weight", cfg.dim, cfg.ffn_dim)}
            if getattr(cfg, "qkv_bias", False):
                L.update(bq=self.vec(b + "attn_q.bias", qd), bk=self.vec(b + "attn_k.bias", kvd),
                         bv=self.vec(b + "attn_v.bias", kvd))
            if getattr(cfg, "qk_norm", False):
                L.update(q_norm=self.vec(b + "attn_q_norm.weight", cfg.head_dim),
                         k_norm=self.vec(b + "attn_k_norm.weight", cfg.head_dim))
            layers.append(L)
        embd = self.mat("token_embd.weight", cfg.vocab, cfg.dim)
        out = self.mat("output.weight", cfg.vocab, cfg.dim) if "output.weight" in self.by_name else embd
        return {"layers": layers, "tok_embd": embd, "out_norm": self.vec("output_norm.weight", cfg.dim), "output": out}

    def load_net(self, eng, max_ctx: int):
        """A hk_amd.net.Net holding this file's decoder, uploaded from the mapped tensor bytes."""
        from .net import Net

        cfg = self.config(max_ctx)
        net = Net(eng, cfg)
        try:
            net.load(self.model(cfg))
        except Exception:
            net.close()
            raise
        return net
