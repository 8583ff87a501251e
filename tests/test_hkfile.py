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
