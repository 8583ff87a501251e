"""hk's block formats on the quantized-linear path: StorageType codes and block geometry.

Codes are hk's StorageType bytes (reference src/format.zig:26-84); geometry is
src/quant/blocks.zig:17-34 and the size table `info` / `byteSize` (blocks.zig:84-127).
"""
from __future__ import annotations

Q4_0 = 0x15
Q8_0 = 0x16
Q4_1 = 0x17
Q5_0 = 0x18
Q5_1 = 0x19
Q4_K = 0x42
Q5_K = 0x43
Q6_K = 0x44
IQ4_NL = 0x55
IQ4_XS = 0x56
# Formats hk decodes to floats before its dots (src/format.zig:71-93).
Q2_K = 0x40
Q3_K = 0x41
IQ1_S = 0x50
IQ1_M = 0x51
IQ2_XXS = 0x52
IQ2_XS = 0x53
IQ3_XXS = 0x54
IQ2_S = 0x57
IQ3_S = 0x58
TQ1_0 = 0x60
TQ2_0 = 0x61
MXFP4 = 0x62
NVFP4 = 0x63
FALLBACK = (Q2_K, Q3_K, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M, TQ1_0, TQ2_0, MXFP4, NVFP4)

NAMES = {Q8_0: "q8_0", Q4_K: "q4_k", Q6_K: "q6_k", IQ4_NL: "iq4_nl",
         Q4_0: "q4_0", Q4_1: "q4_1", Q5_0: "q5_0", Q5_1: "q5_1", Q5_K: "q5_k", IQ4_XS: "iq4_xs",
         Q2_K: "q2_k", Q3_K: "q3_k", IQ2_XXS: "iq2_xxs", IQ2_XS: "iq2_xs", IQ2_S: "iq2_s", IQ3_XXS: "iq3_xxs",
         IQ3_S: "iq3_s", IQ1_S: "iq1_s", IQ1_M: "iq1_m", TQ1_0: "tq1_0", TQ2_0: "tq2_0", MXFP4: "mxfp4",
         NVFP4: "nvfp4"}
BY_NAME = {v: k for k, v in NAMES.items()}

# weights per block, bytes per block (blocks.zig:49-72 size asserts)
INFO = {Q8_0: (32, 34), IQ4_NL: (32, 18), Q4_K: (256, 144), Q6_K: (256, 210),
        Q4_0: (32, 18), Q4_1: (32, 20), Q5_0: (32, 22), Q5_1: (32, 24), Q5_K: (256, 176), IQ4_XS: (256, 136),
        Q2_K: (256, 84), Q3_K: (256, 110), IQ2_XXS: (256, 66), IQ2_XS: (256, 74), IQ2_S: (256, 82),
        IQ3_XXS: (256, 98), IQ3_S: (256, 110), IQ1_S: (256, 50), IQ1_M: (256, 56), TQ1_0: (256, 54),
        TQ2_0: (256, 66), MXFP4: (32, 17), NVFP4: (64, 36)}
# The 32-weight formats (A8 activations), and those of them with an offset m per block.
LEGACY = (Q8_0, IQ4_NL, Q4_0, Q4_1, Q5_0, Q5_1)
WITH_M = (Q4_1, Q5_1)

# Activation kind each format is dotted against (vecdot.zig:185-191).
ACT_A8, ACT_Q8K, ACT_F32 = 0, 1, 2
ACT_KIND = {Q4_K: ACT_Q8K, Q5_K: ACT_Q8K, Q6_K: ACT_Q8K, IQ4_XS: ACT_Q8K, **{t: ACT_A8 for t in LEGACY},
            **{t: ACT_Q8K for t in FALLBACK}, MXFP4: ACT_A8, NVFP4: ACT_F32}

# Bits per weight in the file layout (the numerator of the bandwidth roofline).
BPW = {t: 8.0 * b / e for t, (e, b) in INFO.items()}

# hk's IQ4_NL codebook (src/quant/tables.zig:13).
KVALUES_IQ4NL = (-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113)


class UnsupportedType(ValueError):
    pass


class NotBlockAligned(ValueError):
    pass


def byte_size(t: int, n_elems: int) -> int:
    """Exact bytes of n_elems weights of type t; refuses partial blocks (blocks.zig:123-127)."""
    if t not in INFO:
        raise UnsupportedType(f"storage type 0x{t:02x} is not on the HIP path")
    elems, nbytes = INFO[t]
    if n_elems % elems:
        raise NotBlockAligned(f"{n_elems} weights is not a whole number of {elems}-weight blocks")
    return n_elems // elems * nbytes


def matrix_bytes(t: int, rows: int, cols: int) -> int:
    """Bytes of a rows x cols matrix (abi_ops.zig:56-62)."""
    if t not in INFO:
        raise UnsupportedType(f"storage type 0x{t:02x} is not on the HIP path")
    if cols % INFO[t][0]:
        raise NotBlockAligned(f"cols {cols} is not a whole number of blocks")
    return rows * byte_size(t, cols)
