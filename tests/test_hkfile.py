"""The .hk container reader (hk_amd.hkfile) on files written to the reference's layout
(tests/hkwriter.py): header, metadata and tensor table round trip; tensors are views of the
mapping; the configuration and tensor checks of config.zig / weights.zig; tied output; f16 / bf16
vectors; corrupt files refused."""
from __future__ import annotations

import os

import numpy as np
import pytest

from hk_amd import formats as F
from hk_amd import synth
from hk_amd.hkfile import HkFile, HkFormatError
from hk_amd.net import Config
from tests.hkwriter import write_hk, write_model


def test_round_trip_of_header_metadata_and_table(tmp_path):
    p = str(tmp_path / "t.hk")
    a = np.arange(300, dtype=np.uint8)
    b = np.linspace(-1, 1, 7).astype(np.float32)
    md = {"general.architecture": "llama", "n": 7, "x": 2.5, "flag": True, "s": "hello"}
    write_hk(p, md, [("a", F.Q8_0, (3, 100), a.tobytes()), ("b.vec", 0, (7,), b.tobytes())])
    with HkFile(p) as f:
        assert f.version == (1, 0) and f.tensor_count == 2 and f.metadata == md
        ea = f.entry("a")
        assert ea.t == F.Q8_0 and ea.shape == (3, 100) and ea.data_offset % 128 == 0 and ea.data_size == 300
        assert np.array_equal(f.data("a"), a)
        assert isinstance(f.data("a"), np.memmap)  # a view of the mapping, not a copy
        assert np.array_equal(f.vec("b.vec", 7), b)
        with pytest.raises(HkFormatError):
            f.entry("missing")


def test_config_and_model_from_metadata(tmp_path):
    cfg = Config(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=256, vocab=100, max_ctx=64,
                 rope_neox=True, rope_base=1e6)
    model = synth.model_np(cfg, F.Q4_K, seed=3, out_fmt=F.Q6_K, embd_fmt=F.Q8_0, qk_norm=True)
    p = str(tmp_path / "q3.hk")
    write_model(p, "qwen3", cfg, model, vec_type=1)
    with HkFile(p) as f:
        c = f.config(max_ctx=64)
        assert (c.dim, c.n_layers, c.n_heads, c.n_kv_heads, c.head_dim, c.ffn_dim, c.vocab) == \
               (256, 2, 4, 2, 64, 256, 100)
        assert c.rope_neox and c.qk_norm and not c.qkv_bias and c.rope_base == 1e6
        m = f.model(c)
        raw, t = m["layers"][1]["w_down"]
        assert t == F.Q4_K and np.array_equal(raw, model["layers"][1]["w_down"][0])
        assert np.array_equal(m["layers"][0]["q_norm"], model["layers"][0]["q_norm"].astype(np.float16).astype(np.float32))
        assert m["output"][1] == F.Q6_K
    tied = str(tmp_path / "tied.hk")
    write_model(tied, "llama", cfg, model, tie_output=True, vec_type=2, style_key=False)
    with HkFile(tied) as f:
        c = f.config(max_ctx=64)
        assert not c.rope_neox and not c.qk_norm  # llama: adjacent pairs unless the file says otherwise
        m = f.model(c)
        assert m["output"][1] == F.Q8_0 and np.array_equal(m["output"][0], m["tok_embd"][0])  # tied


def test_refuses_corrupt_files(tmp_path):
    p = str(tmp_path / "bad.hk")
    write_hk(p, {"general.architecture": "llama"}, [("w", F.Q4_K, (2, 256), bytes(288))])
    data = bytearray(open(p, "rb").read())
    bad = bytearray(data)
    bad[0:4] = b"GGUF"
    open(p, "wb").write(bad)
    with pytest.raises(HkFormatError, match="not an hk"):
        HkFile(p)
    open(p, "wb").write(data[:-100])  # the tensor's payload cut short
    with pytest.raises(HkFormatError, match="outside"):
        HkFile(p)
    open(p, "wb").write(data)
    with HkFile(p) as f:
        with pytest.raises(HkFormatError, match="shape"):
            f.mat("w", 2, 512)
        assert f.mat("w", 2, 256)[1] == F.Q4_K
    os.remove(p)


def test_rope_scaling_from_metadata(tmp_path):
    """parseRopeScaling (config.zig:163-223): the type or a bare factor (linear), the original
    context defaulting to the training one, llama3's band and yarn's keys, the rope_freqs.weight
    factors; bad values refused."""
    cfg = Config(dim=256, n_layers=1, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=256, vocab=64, max_ctx=64)
    model = synth.model_np(cfg, F.Q8_0, seed=5, qk_norm=False)
    p = str(tmp_path / "r.hk")
    factors = 1.0 + np.arange(32, dtype=np.float32) / 8
    write_model(p, "llama", cfg, model, rope_freqs=factors,
                extra_meta={"llama.rope.scaling.type": "llama3", "llama.rope.scaling.factor": 8.0,
                            "llama.rope.scaling.original_context_length": 8192, "hk.rope.high_freq_factor": 5.0})
    with HkFile(p) as f:
        c = f.config(max_ctx=64)
        r = c.rope_scaling
        assert (r.kind, r.factor, r.orig_ctx, r.low_freq_factor, r.high_freq_factor) == ("llama3", 8.0, 8192, 1.0, 5.0)
        assert np.array_equal(c.rope_freq_factors, factors)
    write_model(p, "llama", cfg, model, extra_meta={"llama.rope.scaling.factor": 2.0})
    with HkFile(p) as f:
        r = f.config(max_ctx=64).rope_scaling
        assert (r.kind, r.factor, r.orig_ctx) == ("linear", 2.0, 4096)  # bare factor; training context
    write_model(p, "qwen2", cfg, model, extra_meta={"qwen2.rope.scaling.type": "yarn", "qwen2.rope.scaling.factor": 4.0,
                                                     "qwen2.rope.scaling.attn_factor": 0.5, "hk.rope.beta_fast": 16.0})
    with HkFile(p) as f:
        r = f.config(max_ctx=64).rope_scaling
        assert (r.kind, r.factor, r.beta_fast, r.beta_slow, r.attn_factor) == ("yarn", 4.0, 16.0, 1.0, 0.5)
    for bad, msg in (({"llama.rope.scaling.type": "dynamic", "llama.rope.scaling.factor": 2.0}, "not supported"),
                     ({"llama.rope.scaling.type": "linear"}, "needs"),
                     ({"llama.rope.scaling.factor": 0.5}, "at least 1"),
                     ({"llama.rope.scaling.type": "llama3", "llama.rope.scaling.factor": 8.0,
                       "hk.rope.low_freq_factor": 4.0}, "low_freq_factor")):
        write_model(p, "llama", cfg, model, extra_meta=bad)
        with HkFile(p) as f:
            with pytest.raises(HkFormatError, match=msg):
                f.config(max_ctx=64)
    write_model(p, "llama", cfg, model, extra_meta={"llama.attention.sliding_window": 4096})
    with HkFile(p) as f:
        with pytest.raises(HkFormatError, match="sliding window"):
            f.config(max_ctx=64)
    write_model(p, "llama", cfg, model, rope_freqs=-factors)
    with HkFile(p) as f:
        with pytest.raises(HkFormatError, match="positive"):
            f.config(max_ctx=64)


def test_hand_built_container_bytes(tmp_path):
    """A container written byte by byte from the reference's field order, not through
    tests/hkwriter.py: FileHeader (src/format.zig:133-152: magic, versions, flags, alignment,
    split index, counts, offsets and sizes, appendix, checksum, split count, 38 reserved bytes),
    metadata (src/metadata.zig:225-264: key length u16, key, tag u8, value length u32, value) and one
    tensor table entry (src/tensor_toc.zig:39-66: name length u16, name, storage type, tile layout,
    sparsity, ndim, shape u64 x ndim, six u64 offsets / sizes, block size u16, sparsity ratio f32)."""
    header = bytes.fromhex(
        "484b4e54"          # magic "HKNT"
        "0100" "0000"       # version 1.0
        "03000000"          # flags
        "8000" "0000"       # alignment 128, split index 0
        "0100000000000000"  # tensor count 1
        "0200000000000000"  # metadata kv count 2
        "8000000000000000"  # metadata offset 128
        "2000000000000000"  # metadata size 32
        "a000000000000000"  # tensor table offset 160
        "4d00000000000000"  # tensor table size 77
        "0001000000000000"  # tensor data offset 256
        "0000000000000000"  # appendix offset
        "0000000000000000"  # checksum
        "0100"              # split count 1
        + "00" * 38)        # reserved
    metadata = bytes.fromhex(
        "0100" "6e" "02" "08000000" "0700000000000000"  # "n": int64 7
        "0400" "61726368" "01" "05000000" "7177656e33")  # "arch": string "qwen3"
    toc = bytes.fromhex(
        "0100" "74"                                     # name "t"
        "16" "00" "00" "02"                             # Q8_0, tile layout 0, no sparsity, 2 dims
        "0100000000000000" "2000000000000000"           # shape (1, 32)
        "0001000000000000" "2200000000000000"           # data at 256, 34 bytes
        "0000000000000000" "0000000000000000"           # residual offset / size
        "0000000000000000" "0000000000000000"           # scale offset / size
        "2000" "0000c03e")                              # block size 32, sparsity ratio 0.375
    block = bytes.fromhex("003c") + bytes(range(256 - 16, 256)) + bytes(range(16))  # d = 1.0, qs = -16..15
    assert len(header) == 128 and len(metadata) == 32 and len(toc) == 77
    raw = header + metadata + toc + bytes(256 - 237) + block
    p = tmp_path / "hand.hk"
    p.write_bytes(raw)
    with HkFile(str(p)) as f:
        assert f.version == (1, 0) and f.flags == 3 and f.alignment == 128 and f.split_count == 1
        assert f.tensor_count == 1 and f.metadata == {"n": 7, "arch": "qwen3"}
        e = f.entry("t")
        assert (e.t, e.tile_layout, e.sparsity, e.shape) == (F.Q8_0, 0, 0, (1, 32))
        assert (e.data_offset, e.data_size, e.block_size, e.sparsity_ratio) == (256, 34, 32, 0.375)
        assert bytes(f.data("t")) == block
        from oracle import oracle as O
        assert np.array_equal(O.dequantize(F.Q8_0, np.frombuffer(block, np.uint8), 32), np.arange(-16, 16, dtype=np.float32))
    p.write_bytes(raw[:200])  # the tensor table runs past the end
    with pytest.raises(HkFormatError):
        HkFile(str(p))
