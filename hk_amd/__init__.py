"""hk_amd: MI355X (gfx950) HIP engine for hk's quantized-linear hot path and the network pass
around it, behind the C ABI of include/hkhip.h (libhkhip.so).

Kernels: the activation quantizers (qact: hk's A8 and Q8K), decode products for 1-8 tokens
(register-streamed integer dots; small-batch MFMA for Q4_K / Q6_K), prefill GEMMs on int8 MFMA, and a
float-decode path, over every hk block format (Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_NL,
IQ4_XS; Q2_K, Q3_K, the IQ1 / IQ2 / IQ3 families, TQ1_0, TQ2_0, MXFP4, NVFP4). hk_amd.net runs whole
decoders on them with hk's engine contract (passes over several sequences' cache slots, logits of
chosen rows, partial offload, the planner's size estimate); hk_amd.hkfile reads .hk containers.
"""
from . import formats  # noqa: F401
from ._lib import HipError, lib  # noqa: F401
from .engine import ACCUMULATE, SILU_MUL, STORE, DevMat, Engine, gemm, gemv  # noqa: F401
