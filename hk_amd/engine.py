"""Python host side of the HIP engine, shaped like hk's device-engine operator interface.

The reference's CUDA engine multiplies a device matrix by prepared activations with
``prepare(x, count, n, mats)`` then ``mm(m, x, y, n)`` (src/cuda/engine.zig:581-630) over
``DevMat{mem, t, rows, cols}`` (engine.zig:111-116) uploaded by ``upload`` (493-506). This
module exposes the same operations over the C ABI (include/hkhip.h); device buffers are torch
tensors on ``cuda:<device>`` (torch is only the allocator and stream here) or raw pointers.

The host-pointer products ``gemm`` / ``gemv`` mirror src/engine/abi_ops.zig:65-107 and the
C ABI ``hk_gemv_*`` (src/c_api.zig:1380-1400): NumPy in, NumPy out, NaN-filled on failure.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import formats
from ._lib import HipError, HkhipMat, check, lib

STORE, ACCUMULATE, SILU_MUL = 0, 1, 2  # output modes (hkhip.h HKHIP_STORE / ACCUMULATE / SILU_MUL)
MIN_TILED_TOKENS = 8  # matmul.zig:18


def _ptr(x) -> int | None:
    """Device pointer of a torch tensor, an int, or None."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


@dataclass
class DevMat:
    """A weight matrix resident on the device (DevMat in src/cuda/engine.zig:111-116)."""
    raw: HkhipMat

    @property
    def t(self) -> int:
        return self.raw.t

    @property
    def rows(self) -> int:
        return self.raw.rows

    @property
    def cols(self) -> int:
        return self.raw.cols

    @property
    def file_bytes(self) -> int:
        return self.raw.file_bytes


class Engine:
    """One device and one stream (Engine in src/cuda/engine.zig)."""

    def __init__(self, device: int = 0, stream: int | None = None):
        self._h = ctypes.c_void_p()
        check(lib().hkhip_init(device, ctypes.byref(self._h)))
        self.device = device
        self._mats: list[HkhipMat] = []
        if stream is not None:
            self.set_stream(stream)

    # -- lifetime ------------------------------------------------------------------------
    def close(self) -> None:
        if self._h:
            for m in self._mats:
                lib().hkhip_free(self._h, ctypes.byref(m))
            self._mats.clear()
            lib().hkhip_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def name(self) -> str:
        return lib().hkhip_device_name(self._h).decode()

    def set_stream(self, stream: int | None) -> None:
        """Run on an existing hipStream_t, e.g. torch.cuda.current_stream().cuda_stream
        (0 / None is the null stream); use_own_stream() goes back to the engine's stream."""
        check(lib().hkhip_set_stream(self._h, stream or None))

    def use_own_stream(self) -> None:
        check(lib().hkhip_use_own_stream(self._h))

    @property
    def stream(self) -> int:
        return lib().hkhip_stream(self._h) or 0

    def sync(self) -> None:
        check(lib().hkhip_sync(self._h))

    # -- weights -------------------------------------------------------------------------
    @staticmethod
    def supports(t: int) -> bool:
        return bool(lib().hkhip_supports(t))

    def upload(self, data, t: int, rows: int, cols: int) -> DevMat:
        """Copies hk-file-layout weights (a NumPy uint8 buffer, e.g. an mmap view, or a device
        tensor) to the device in the engine's layout (Engine.upload, cuda/engine.zig:493-506)."""
        m = HkhipMat()
        if isinstance(data, np.ndarray):
            buf = np.ascontiguousarray(data).view(np.uint8)
            rc = lib().hkhip_upload(self._h, buf.ctypes.data, buf.nbytes, t, rows, cols, 0, ctypes.byref(m))
        else:
            nbytes = data.numel() * data.element_size()
            rc = lib().hkhip_upload(self._h, _ptr(data), nbytes, t, rows, cols, 1, ctypes.byref(m))
        check(rc)
        self._mats.append(m)
        return DevMat(m)

    def free(self, m: DevMat) -> None:
        lib().hkhip_free(self._h, ctypes.byref(m.raw))
        self._mats = [x for x in self._mats if x is not m.raw]

    def dequantize(self, m: DevMat, out, row0: int = 0, nrows: int | None = None) -> None:
        """Bit-exact f32 decode of rows into `out` (device, [nrows][cols])."""
        nrows = m.rows - row0 if nrows is None else nrows
        check(lib().hkhip_dequantize(self._h, ctypes.byref(m.raw), row0, nrows, _ptr(out)))

    # -- activations ---------------------------------------------------------------------
    @staticmethod
    def act_bytes(n: int, k: int) -> int:
        return int(lib().hkhip_act_bytes(n, k))

    def qact(self, x, n: int, k: int, kind: int, xq) -> None:
        check(lib().hkhip_qact(self._h, _ptr(x), n, k, kind, _ptr(xq)))

    def prepare(self, x, n: int, k: int, mats, xq) -> None:
        """Quantizes x [n][k] once for every kind the products in `mats` read
        (prepare: cuda/engine.zig:614-630; Cpu.prepare: cpu_backend.zig:214-225)."""
        for kind in sorted({formats.ACT_KIND[m.t] for m in mats} - {formats.ACT_F32}):
            self.qact(x, n, k, kind, xq)

    def act_export(self, xq, n: int, k: int, kind: int) -> np.ndarray:
        """The prepared activations as hk's block structs (BlockA8 / BlockQ8K bytes)."""
        nb = n * k // (32 if kind == formats.ACT_A8 else 256)
        out = np.zeros(nb * (40 if kind == formats.ACT_A8 else 292), np.uint8)
        check(lib().hkhip_act_export(self._h, _ptr(xq), n, k, kind, out.ctypes.data))
        return out

    # -- products ------------------------------------------------------------------------
    def matvec(self, m: DevMat, xq, y, n: int, bias=None, mode: int = STORE) -> None:
        check(lib().hkhip_matvec(self._h, ctypes.byref(m.raw), _ptr(xq), _ptr(y), n, _ptr(bias), mode))

    def matvec_parts(self, mats, ys, n: int, x=None, xq=None, biases=None, mode: int = STORE) -> None:
        """Up to four matrices sharing one input in one launch (matmul.runParts). Pass the f32
        input `x` (quantized inside the kernel) or a prepared `xq`."""
        k = len(mats)
        arr = (HkhipMat * k)(*[m.raw for m in mats])
        yp = (ctypes.c_void_p * k)(*[_ptr(y) for y in ys])
        bp = None if biases is None else (ctypes.c_void_p * k)(*[_ptr(b) for b in biases])
        check(lib().hkhip_matvec_parts(self._h, arr, k, _ptr(x), _ptr(xq), n, yp, bp, mode))

    def matvec_parts_rmsnorm(self, mats, ys, n: int, x, norm, eps: float, biases=None, mode: int = STORE) -> None:
        """matvec_parts on rmsnorm(x) * norm, the norm fused into the products' input staging."""
        k = len(mats)
        arr = (HkhipMat * k)(*[m.raw for m in mats])
        yp = (ctypes.c_void_p * k)(*[_ptr(y) for y in ys])
        bp = None if biases is None else (ctypes.c_void_p * k)(*[_ptr(b) for b in biases])
        check(lib().hkhip_matvec_parts_rmsnorm(self._h, arr, k, _ptr(x), _ptr(norm), eps, n, yp, bp, mode))

    def gemm(self, m: DevMat, xq, y, n: int, bias=None, mode: int = STORE) -> None:
        check(lib().hkhip_gemm(self._h, ctypes.byref(m.raw), _ptr(xq), _ptr(y), n, _ptr(bias), mode))

    def mm(self, m: DevMat, xq, y, n: int, bias=None, mode: int = STORE) -> None:
        """y[t][r] = dot(W[r], x[t]) + bias[r]: decode kernel up to 8 tokens, 8-token decode passes
        up to the GEMM's break-even (Q6_K / Q8_0 32, IQ4_NL 24 tokens), MFMA GEMM beyond
        (mm: cuda/engine.zig:581-611; matmul.zig:18,107)."""
        check(lib().hkhip_mm(self._h, ctypes.byref(m.raw), _ptr(xq), _ptr(y), n, _ptr(bias), mode))

    def mm_noalloc(self, m: DevMat, x, y, n: int, bias=None, mode: int = STORE) -> None:
        """mm on an f32 input x [n][cols], quantized into the library's fixed activation buffer:
        allocates nothing (for callers that cannot). Calls on one device share that buffer."""
        check(lib().hkhip_mm_noalloc(self._h, ctypes.byref(m.raw), _ptr(x), _ptr(y), n, _ptr(bias), mode))


# -- host-pointer products (abi_ops.gemm / gemv, c_api hk_gemv_*) ---------------------------

def gemm(t: int, w: np.ndarray, x: np.ndarray, bias: np.ndarray | None, m: int, k: int, n: int) -> np.ndarray:
    """y[n][m] = W x + bias with host arrays, on device 0 (abi_ops.zig:65-103).
    Raises HipError on failure; the output buffer the C ABI filled is NaN then."""
    w = np.ascontiguousarray(w).view(np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    y = np.empty((n, m), np.float32)
    rc = lib().hkhip_gemm_host(t, w.ctypes.data, x.ctypes.data, None if b is None else b.ctypes.data,
                               y.ctypes.data, m, k, n)
    if rc < 0:
        err = HipError(rc, (lib().hkhip_last_error() or b"").decode())
        err.y = y
        raise err
    return y


def gemv(t: int, w: np.ndarray, x: np.ndarray, bias: np.ndarray | None, m: int, k: int) -> np.ndarray:
    """y[m] = W x + bias (abi_ops.zig:105-107, hk_gemv_*)."""
    return gemm(t, w, x, bias, m, k, 1)[0]
