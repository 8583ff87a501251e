"""hk_amd: MI355X (gfx950) HIP engine for hk's quantized-linear hot path.

Kernels: qact (activation quantizers), mmvq (decode matvec, 1..8 tokens) and mm (prefill
GEMM on int8 MFMA) over hk's Q8_0, Q4_K, Q6_K and IQ4_NL blocks, behind the C ABI of
include/hkhip.h (libhkhip.so).
"""
from . import formats  # noqa: F401
from ._lib import HipError, lib  # noqa: F401
from .engine import ACCUMULATE, SILU_MUL, STORE, DevMat, Engine, gemm, gemv  # noqa: F401
