"""Writes .hk containers for the tests (the reference's writer is Zig and not buildable here):
header src/format.zig:174-199, metadata src/metadata.zig:225-266 serialize, tensor table
src/tensor_toc.zig:39-66 serialize, tensor payloads 128-byte aligned (format.zig ALIGNMENT_BYTES)."""
from __future__ import annotations

import struct

import numpy as np

from hk_amd.hkfile import HEADER, MAGIC, VAL_BOOL, VAL_FLOAT64, VAL_INT64, VAL_STRING


def _meta(md: dict) -> bytes:
    out = b""
    for k, v in md.items():
        kb = k.encode()
        out += struct.pack("<H", len(kb)) + kb
        if isinstance(v, bool):
            out += struct.pack("<BI", VAL_BOOL, 1) + bytes([int(v)])
        elif isinstance(v, int):
            out += struct.pack("<BIq", VAL_INT64, 8, v)
        elif isinstance(v, float):
            out += struct.pack("<BId", VAL_FLOAT64, 8, v)
        else:
            vb = str(v).encode()
            out += struct.pack("<BI", VAL_STRING, len(vb)) + vb
    return out


def write_hk(path: str, metadata: dict, tensors: list) -> None:
    """tensors: (name, storage type, shape, payload bytes)."""
    align = 128
    meta = _meta(metadata)
    meta_off = HEADER.size
    toc_off = meta_off + len(meta)

    def toc_bytes(offsets):
        out = b""
        for (name, t, shape, payload), off in zip(tensors, offsets):
            nb = name.encode()
            out += struct.pack("<H", len(nb)) + nb + struct.pack("<BBBB", t, 0, 0, len(shape))
            out += b"".join(struct.pack("<Q", d) for d in shape)
            out += struct.pack("<QQQQQQ", off, len(payload), 0, 0, 0, 0) + struct.pack("<Hf", 32, 0.0)
        return out

    toc_size = len(toc_bytes([0] * len(tensors)))
    data_off = (toc_off + toc_size + align - 1) // align * align
    offsets, pos = [], data_off
    for _, _, _, payload in tensors:
        offsets.append(pos)
        pos = (pos + len(payload) + align - 1) // align * align
    header = HEADER.pack(MAGIC, 1, 0, 1 | (1 << 4), align, 0, len(tensors), len(metadata), meta_off, len(meta),
                         toc_off, toc_size, data_off, 0, 0, 1, bytes(38))
    with open(path, "wb") as f:
        f.write(header + meta + toc_bytes(offsets))
        for (_, _, _, payload), off in zip(tensors, offsets):
            f.seek(off)
            f.write(bytes(payload))
        f.truncate(pos)


def write_model(path: str, arch: str, cfg, model: dict, tie_output: bool = False, vec_type: int = 0,
                style_key: bool = True, extra_meta: dict | None = None, rope_freqs=None) -> None:
    """A decoder in hk's tensor naming (weights.zig:96-176) and metadata keys (config.zig:225-320).
    vec_type: 0 f32, 1 f16 or 2 bf16 for the norm and bias vectors; style_key: write hk.rope_style
    (else the architecture's default applies); extra_meta: more keys (rope scaling); rope_freqs:
    the rope_freqs.weight tensor (f32)."""
    md = {"general.architecture": arch, f"{arch}.embedding_length": cfg.dim, f"{arch}.block_count": cfg.n_layers,
          f"{arch}.feed_forward_length": cfg.ffn_dim, f"{arch}.attention.head_count": cfg.n_heads,
          f"{arch}.attention.head_count_kv": cfg.n_kv_heads, f"{arch}.attention.key_length": cfg.head_dim,
          f"{arch}.rope.dimension_count": cfg.rope_dim or cfg.head_dim, f"{arch}.rope.freq_base": float(cfg.rope_base),
          f"{arch}.attention.layer_norm_rms_epsilon": float(cfg.rms_eps), f"{arch}.context_length": 4096,
          }
    if style_key:
        md["hk.rope_style"] = "neox" if cfg.rope_neox else "norm"
    md.update(extra_meta or {})

    def vec(v):
        v = np.asarray(v, np.float32)
        if vec_type == 1:
            return 1, v.astype(np.float16).tobytes()
        if vec_type == 2:
            return 2, (v.view(np.uint32) >> 16).astype(np.uint16).tobytes()
        return 0, v.tobytes()

    ts = []

    def add_mat(name, m, rows, cols):
        raw, t = m
        ts.append((name, t, (rows, cols), np.ascontiguousarray(raw).tobytes()))

    def add_vec(name, v):
        t, b = vec(v)
        ts.append((name, t, (len(v),), b))

    qd, kvd = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
    add_mat("token_embd.weight", model["tok_embd"], cfg.vocab, cfg.dim)
    add_vec("output_norm.weight", model["out_norm"])
    if rope_freqs is not None:
        f = np.asarray(rope_freqs, np.float32)
        ts.append(("rope_freqs.weight", 0, (len(f),), f.tobytes()))
    if not tie_output:
        add_mat("output.weight", model["output"], cfg.vocab, cfg.dim)
    for i, L in enumerate(model["layers"]):
        b = f"blk.{i}."
        add_vec(b + "attn_norm.weight", L["attn_norm"])
        add_mat(b + "attn_q.weight", L["wq"], qd, cfg.dim)
        add_mat(b + "attn_k.weight", L["wk"], kvd, cfg.dim)
        add_mat(b + "attn_v.weight", L["wv"], kvd, cfg.dim)
        add_mat(b + "attn_output.weight", L["wo"], cfg.dim, qd)
        add_vec(b + "ffn_norm.weight", L["ffn_norm"])
        add_mat(b + "ffn_gate.weight", L["w_gate"], cfg.ffn_dim, cfg.dim)
        add_mat(b + "ffn_up.weight", L["w_up"], cfg.ffn_dim, cfg.dim)
        add_mat(b + "ffn_down.weight", L["w_down"], cfg.dim, cfg.ffn_dim)
        for k, n in (("bq", "attn_q.bias"), ("bk", "attn_k.bias"), ("bv", "attn_v.bias"),
                     ("q_norm", "attn_q_norm.weight"), ("k_norm", "attn_k_norm.weight")):
            if L.get(k) is not None:
                add_vec(b + n, L[k])
    write_hk(path, md, ts)
