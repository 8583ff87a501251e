"""Shared helpers for the parity tests (the oracle is only used here, as the checker)."""
from __future__ import annotations

import os
import struct

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_fixture(name: str):
    """hk's quant fixture layout (reference tools/gen_quant_fixtures.py:8-11):
    u32 ggml_type, rows, blocks_per_row, block_elems, block_bytes; raw blocks; f32 values."""
    b = open(os.path.join(GOLDEN, f"{name}.bin"), "rb").read()
    gt, rows, bpr, el, bb = struct.unpack("<5I", b[:20])
    nraw = rows * bpr * bb
    raw = np.frombuffer(b[20:20 + nraw], np.uint8).reshape(rows, bpr * bb)
    exp = np.frombuffer(b[20 + nraw:20 + nraw + rows * bpr * el * 4], "<f4").reshape(rows, bpr * el)
    return dict(ggml_type=gt, rows=rows, blocks_per_row=bpr, block_elems=el, block_bytes=bb, raw=raw, expected=exp)


def parity_err(got: np.ndarray, want: np.ndarray) -> float:
    """max |got - want| / max(|want|, 1e-3 * max|want|): relative error with a floor of
    1e-3 of the output's largest magnitude, because pure per-element relative error is
    ill-posed for outputs near zero."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    floor = 1e-3 * max(float(np.max(np.abs(want))), 1e-30)
    return float(np.max(np.abs(got - want) / np.maximum(np.abs(want), floor)))


PARITY_TOL = 1e-3  # max relative error 1e-3 against hk's CPU kernels


def tie_rows(k: int) -> np.ndarray:
    """Activations on which round-half-away and round-half-even disagree, with hand-checkable
    quantized values (reference vecdot.zig:134-148, 150-180: Zig's @round rounds half away).

    Every 32-value block starts with -127, so amax = 127: the A8 scale is d = 127/127 = 1 and
    1/d = 1 exactly, and for Q8K the signed max of every 256-block is -127, so iscale =
    -127/-127 = 1. Then q = round(x) exactly, and the other values k + 0.5 (k = -15..14) are ties:
    round-half-away gives k + 1 for k >= 0 and k for k < 0; rint would give the even neighbour.
    Returns x [1][k] and the expected q [1][k] (int64)."""
    blk = np.concatenate([[-127.0], np.arange(-15, 16) + 0.5]).astype(np.float32)  # 32 values
    x = np.tile(blk, k // 32)[None, :]
    q = np.where(x >= 0, np.floor(x) + 1, np.ceil(x) - 1).astype(np.int64)  # away from zero
    q[:, ::32] = -127
    return x, q
