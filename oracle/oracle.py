"""ctypes view of the CPU oracle (oracle/hk_oracle.c). TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg import this
module, and only as the checker or the timed CPU baseline. The HIP product path never
calls it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhk_oracle.so")

Q8_0, Q4_K, Q6_K, IQ4_NL = 0x16, 0x42, 0x44, 0x55
Q4_0, Q4_1, Q5_0, Q5_1 = 0x15, 0x17, 0x18, 0x19
Q5_K, IQ4_XS = 0x43, 0x56
_A8 = (Q8_0, IQ4_NL, Q4_0, Q4_1, Q5_0, Q5_1)

A8_DTYPE = np.dtype([("d", "<f4"), ("s", "<i4"), ("qs", "i1", (32,))])  # vecdot.zig:22-26
Q8K_DTYPE = np.dtype([("d", "<f4"), ("qs", "i1", (256,)), ("bsums", "<i2", (16,))])  # blocks.zig:25
assert A8_DTYPE.itemsize == 40 and Q8K_DTYPE.itemsize == 292


def build() -> None:
    """Compile the oracle with its Makefile (gcc only)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P, S, F, I = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_float, ctypes.c_int
        L.hko_dequantize_row.argtypes = [I, P, S, P, S]
        L.hko_quantize_a8.argtypes = [P, S, P]
        L.hko_quantize_q8k.argtypes = [P, S, P]
        L.hko_dot_row.argtypes = [I, P, S, P, P]
        L.hko_dot_row.restype = F
        L.hko_scales_mins_k4_words.argtypes = [P, P, P]
        L.hko_scale_min_k4.argtypes = [I, P, P, P]
        L.hko_matmul.argtypes = [I, P, S, S, P, S, P, P, I]
        L.hko_matmul_path.argtypes = [I, P, S, S, P, S, P, P, I, I]
        L.hko_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.hko_f16_to_f32.restype = F
        L.hko_block_elems.argtypes = [I]
        L.hko_block_bytes.argtypes = [I]
        L.hko_act_kind.argtypes = [I]
        L.hkc_pick_level.argtypes = [ctypes.c_char_p]
        L.hkc_pick_level.restype = I
        L.hkc_level_name.argtypes = [I]
        L.hkc_level_name.restype = ctypes.c_char_p
        L.hkc_matvec_q4k.argtypes = [I, P, S, S, P, P, I]
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def block_elems(t: int) -> int:
    e = lib().hko_block_elems(t)
    if not e:
        raise KeyError(t)
    return e


def block_bytes(t: int) -> int:
    b = lib().hko_block_bytes(t)
    if not b:
        raise KeyError(t)
    return b


def act_kind(t: int) -> int:
    """0 = A8 (per 32), 1 = Q8K (per 256), 2 = f32; vecdot.zig:185-191."""
    return lib().hko_act_kind(t)


def dequantize(t: int, raw: np.ndarray, n: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(n, np.float32)
    rc = lib().hko_dequantize_row(t, _p(raw), raw.size, _p(out), n)
    if rc != 0:
        raise ValueError("bad length or type")
    return out


def quantize_a8(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // 32, A8_DTYPE)
    lib().hko_quantize_a8(_p(x), x.size, _p(out))
    return out


def quantize_q8k(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // 256, Q8K_DTYPE)
    lib().hko_quantize_q8k(_p(x), x.size, _p(out))
    return out


def dot_row(t: int, row: np.ndarray, act: np.ndarray) -> float:
    row = np.ascontiguousarray(row, dtype=np.uint8)
    k = row.size // block_bytes(t) * block_elems(t)
    if act_kind(t) == 0:
        return lib().hko_dot_row(t, _p(row), k, _p(act), None)
    return lib().hko_dot_row(t, _p(row), k, None, _p(act))


def matmul(t: int, w: np.ndarray, m: int, k: int, x: np.ndarray, n: int,
           bias: np.ndarray | None = None, threads: int = 1, tiled: bool | None = None) -> np.ndarray:
    """y[n][m] = W x + bias as hk's CPU engine computes it (abi_ops.gemm)."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty((n, m), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    if tiled is None:
        rc = lib().hko_matmul(t, _p(w), m, k, _p(x), n, _p(b), _p(y), threads)
    else:
        rc = lib().hko_matmul_path(t, _p(w), m, k, _p(x), n, _p(b), _p(y), threads, int(tiled))
    if rc != 0:
        raise ValueError(f"oracle matmul failed: {rc}")
    return y


def scales_mins_words(packed: np.ndarray):
    p = np.ascontiguousarray(packed, np.uint8)
    sc = np.zeros(8, np.uint8)
    mn = np.zeros(8, np.uint8)
    lib().hko_scales_mins_k4_words(_p(p), _p(sc), _p(mn))
    return sc, mn


def scale_min_k4(j: int, packed: np.ndarray):
    p = np.ascontiguousarray(packed, np.uint8)
    sc = ctypes.c_uint8()
    mn = ctypes.c_uint8()
    lib().hko_scale_min_k4(j, _p(p), ctypes.byref(sc), ctypes.byref(mn))
    return sc.value, mn.value


# -- hk's SIMD decode kernel (hk_cpu_simd.c): the benchmark's CPU baseline --------------------

SIMD_LEVELS = ("avx512-vnni", "avx2-vnni", "avx2", "generic")


def simd_level(name: str | None = None) -> int:
    """The instruction-set level hk would run here (kernels.zig:55-85), or the named one; -1 if
    the processor lacks it."""
    return lib().hkc_pick_level(None if name is None else name.encode())


def simd_level_name(level: int) -> str:
    return lib().hkc_level_name(level).decode()


def matvec_q4k_simd(w: np.ndarray, m: int, k: int, x: np.ndarray, threads: int = 1,
                    level: int | None = None) -> np.ndarray:
    """y = W x for a Q4_K matrix and one token through hk's SIMD kernel at `level`."""
    lv = simd_level() if level is None else level
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    y = np.empty(m, np.float32)
    if lib().hkc_matvec_q4k(lv, _p(w), m, k, _p(x), _p(y), threads) != 0:
        raise ValueError(f"hkc_matvec_q4k failed (level {lv})")
    return y
