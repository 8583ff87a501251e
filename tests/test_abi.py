"""The C-ABI library without a GPU: it loads, exports exactly what include/hkhip.h declares,
and its host-side logic (sizes, validation, error codes, NaN poisoning) behaves as the
reference's C ABI does. No compute call reaches a device here."""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest

from hk_amd import _lib, formats as F

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions() -> set[str]:
    text = open(os.path.join(ROOT, "include", "hkhip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(hkhip_\w+)\s*\(", text))


def test_library_builds_and_loads():
    assert os.path.exists(_lib.LIB_PATH), "run __graft_entry__.build() first"
    _lib.lib()


def test_every_declared_symbol_is_exported_and_bound():
    declared = header_functions()
    assert len(declared) >= 25
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for name in sorted(declared):
        assert hasattr(lib, name), f"{name} declared in hkhip.h but not exported"
    assert declared == set(_lib.SIGNATURES), "Python binding and header disagree"


def test_missing_library_fails_loudly(monkeypatch):
    monkeypatch.setattr(_lib, "LIB_PATH", "/nonexistent/libhkhip.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="missing"):
        _lib.lib()


def test_sizes_match_the_block_table():
    L = _lib.lib()
    for t, (elems, nbytes) in F.INFO.items():
        assert L.hkhip_supports(t) == 1
        assert L.hkhip_matrix_bytes(t, 7, elems * 3) == 7 * 3 * nbytes
        assert F.matrix_bytes(t, 7, elems * 3) == 7 * 3 * nbytes
    assert L.hkhip_matrix_bytes(F.Q4_K, 14336, 4096) == 33030144
    assert L.hkhip_matrix_bytes(F.Q6_K, 128256, 4096) == 430940160
    assert L.hkhip_supports(0x01) == 0  # f16 is not on this path
    assert L.hkhip_matrix_bytes(0x01, 1, 256) == -1  # UNSUPPORTED_TYPE
    assert L.hkhip_matrix_bytes(F.Q4_K, 1, 100) == -2  # UNSUPPORTED_SHAPE
    assert b"whole number" in L.hkhip_last_error()


def test_byte_size_rejects_partial_blocks():
    """blocks.zig:129-134 ('block size table matches the reference')."""
    with pytest.raises(F.NotBlockAligned):
        F.byte_size(F.Q4_K, 100)
    with pytest.raises(F.UnsupportedType):
        F.byte_size(0x22, 256)
    assert F.BPW[F.Q4_K] == 4.5 and F.BPW[F.Q6_K] == 6.5625 and F.BPW[F.Q8_0] == 8.5


def test_act_bytes_holds_both_kinds():
    L = _lib.lib()
    n, k = 3, 4096
    need = n * k * 2 + n * k // 32 * 8 + n * k // 256 * 4 + n * k // 16 * 2
    assert L.hkhip_act_bytes(n, k) >= need
    assert L.hkhip_act_bytes(n, k) % 256 == 0


def test_host_product_poisons_output_on_failure():
    """A failing hkhip_gemv_* fills y with NaN (c_api.zig:16-18) and returns a negative code.
    Here it fails either on the bad shape or, on a machine without a GPU, on the device."""
    L = _lib.lib()
    y = np.zeros(4, np.float32)
    w = np.zeros(4 * 144, np.uint8)
    x = np.zeros(100, np.float32)
    rc = L.hkhip_gemv_q4_k(w.ctypes.data, x.ctypes.data, None, y.ctypes.data, 4, 100)
    assert rc == -2 and np.isnan(y).all()


def test_engine_init_reports_missing_device():
    """Without a HIP device, init fails with NO_DEVICE and a message (probeCuda's 'no device')."""
    L = _lib.lib()
    if L.hkhip_device_count() > 0:
        pytest.skip("a device is present")
    h = ctypes.c_void_p()
    assert L.hkhip_init(0, ctypes.byref(h)) == -6
    assert L.hkhip_last_error()


def test_network_bytes_needed_host_logic():
    """hkhip_net_bytes_needed / hkhip_net_layer_bytes are host arithmetic (no device): the planner's
    linear estimate base + n_ctx * per_ctx (backend.zig:92-126 probeCuda: bytesNeeded at n_ctx 0 and
    1) never falls below the real figure; a second slot costs exactly its caches (keys, values and
    the transposed values); a partial network holds only its layers (no embedding, norm or output);
    unsupported shapes give 0."""
    from hk_amd import formats as F, synth
    from hk_amd.net import Config, Options, bytes_needed, layer_bytes

    def cfg(ctx, **kw):
        return Config(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=300, max_ctx=ctx, **kw)

    model = synth.model_np(cfg(1), F.Q4_K, seed=11, out_fmt=F.Q6_K, embd_fmt=F.Q8_0, qk_norm=True, bias=True)
    base, one = bytes_needed(cfg(0), model), bytes_needed(cfg(1), model)
    assert base > 0 and one > base
    for ctx in (7, 64, 100, 1000, 4096):
        assert base + ctx * (one - base) >= bytes_needed(cfg(ctx), model), ctx
    ctx = 1000
    kv = 2 * 2 * 64  # layers x kv heads x head_dim
    vt = (ctx + 31) // 32 * 32
    assert bytes_needed(cfg(ctx), model, Options(slots=2)) - bytes_needed(cfg(ctx), model, Options(slots=1)) == \
        kv * 2 * (2 * ctx + vt)
    full = bytes_needed(cfg(ctx), model, Options(n_batch=64))
    part = bytes_needed(cfg(ctx), model, Options(n_batch=64, layers=1))
    lb = [layer_bytes(cfg(ctx), l) for l in model["layers"]]
    assert all(b > 0 for b in lb)
    io = F.matrix_bytes(F.Q8_0, 300, 256) + 4 * 256 + F.matrix_bytes(F.Q6_K, 300, 256)  # file bytes of the I/O tensors
    assert full - part >= lb[1] + io  # the second layer, the I/O tensors (device layouts at least their file bytes), its caches
    bad = cfg(ctx)
    bad.head_dim = 96
    assert bytes_needed(bad, model) == 0


def test_items_pack_as_the_c_struct():
    """hk_amd.net packs (seq, token, pos) items in bulk into hkhip_item's 16-byte layout (u64 seq,
    u32 token, u32 pos): the bytes match ctypes' own Item structures, for tuples, lists and an
    [n][3] array, with seq ids over the whole u64 range; a value out of its field's range raises."""
    from hk_amd.net import _items

    items = [(2**64 - 1, 5, 7), (0, 2**32 - 1, 0), (3, np.uint32(9), 10)]
    want = (_lib.Item * 3)(*[_lib.Item(*it) for it in items])
    for form in (items, [list(it) for it in items]):
        p, n, keep = _items(form)
        assert n == 3 and ctypes.string_at(p, 48) == bytes(want)
    arr = np.array([[1, 2, 3], [4, 5, 6]], dtype=np.int64)
    p, n, keep = _items(arr)
    assert n == 2 and ctypes.string_at(p, 32) == bytes((_lib.Item * 2)(_lib.Item(1, 2, 3), _lib.Item(4, 5, 6)))
    assert _items([])[1] == 0
    with pytest.raises((OverflowError, ValueError)):
        _items([(-1, 0, 0)])
