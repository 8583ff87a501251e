"""ctypes binding of libhkhip.so (the C ABI declared in include/hkhip.h).

There is no fallback: when the library is missing or cannot be loaded, every entry point of
this package raises. The binding below is the same one hk's Python package would add beside its
libhk binding (reference python/hk/native.py:50-70).
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhkhip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "hkhip.h")


class HipError(RuntimeError):
    """A negative HKHIP_E_* return code, with hkhip_last_error()'s message."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"hkhip error {code}: {msg}")
        self.code = code


class HkhipMat(ctypes.Structure):
    _fields_ = [
        ("mem", ctypes.c_void_p),
        ("file_bytes", ctypes.c_uint64),
        ("dev_bytes", ctypes.c_uint64),
        ("rows", ctypes.c_uint32),
        ("cols", ctypes.c_uint32),
        ("t", ctypes.c_uint8),
        ("owned", ctypes.c_uint8),
        ("pad", ctypes.c_uint8 * 6),
    ]


class NetConfig(ctypes.Structure):
    """hkhip_net_config."""
    _fields_ = [(n, ctypes.c_uint32) for n in ("dim", "n_layers", "n_heads", "n_kv_heads", "head_dim", "ffn_dim",
                                                  "vocab", "rope_dim", "rope_neox", "max_ctx")] + \
               [("rms_eps", ctypes.c_float), ("rope_base", ctypes.c_float), ("inv_freq", ctypes.c_void_p),
                ("rope_mscale", ctypes.c_float)]


class NetTensor(ctypes.Structure):
    """hkhip_net_tensor: hk file-layout bytes in host memory (data NULL: absent)."""
    _fields_ = [("data", ctypes.c_void_p), ("bytes", ctypes.c_uint64), ("t", ctypes.c_uint8)]


class NetOptions(ctypes.Structure):
    """hkhip_net_options (src/cuda/engine.zig:43-58 Options)."""
    _fields_ = [(n, ctypes.c_uint32) for n in ("slots", "layers", "n_batch", "attn_merge_max", "attn_gqa")]


class Item(ctypes.Structure):
    """hkhip_item (src/engine/kv.zig:22-29 Item): {sequence, token, position}."""
    _fields_ = [("seq", ctypes.c_uint64), ("token", ctypes.c_uint32), ("pos", ctypes.c_uint32)]


NET_LAYER_FIELDS = ("attn_norm", "wq", "wk", "wv", "bq", "bk", "bv", "q_norm", "k_norm", "wo", "ffn_norm",
                    "w_gate", "w_up", "w_down")


class NetLayer(ctypes.Structure):
    """hkhip_net_layer."""
    _fields_ = [(n, NetTensor) for n in NET_LAYER_FIELDS]


_P, _U8, _U32, _U64, _I = ctypes.c_void_p, ctypes.c_uint8, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int
_FP = ctypes.POINTER(ctypes.c_float)
_MP = ctypes.POINTER(HkhipMat)

# name -> (restype, argtypes); every function include/hkhip.h declares.
SIGNATURES = {
    "hkhip_device_count": (_I, []),
    "hkhip_init": (_I, [_I, ctypes.POINTER(_P)]),
    "hkhip_destroy": (None, [_P]),
    "hkhip_set_stream": (_I, [_P, _P]),
    "hkhip_use_own_stream": (_I, [_P]),
    "hkhip_stream": (_P, [_P]),
    "hkhip_sync": (_I, [_P]),
    "hkhip_last_error": (ctypes.c_char_p, []),
    "hkhip_device_name": (ctypes.c_char_p, [_P]),
    "hkhip_supports": (_I, [_U8]),
    "hkhip_matrix_bytes": (ctypes.c_int64, [_U8, _U32, _U32]),
    "hkhip_act_bytes": (_U64, [_U32, _U32]),
    "hkhip_alloc": (_I, [_P, _U64, ctypes.POINTER(_P)]),
    "hkhip_dev_free": (None, [_P, _P]),
    "hkhip_copy_h2d": (_I, [_P, _P, _P, _U64]),
    "hkhip_copy_d2h": (_I, [_P, _P, _P, _U64]),
    "hkhip_upload": (_I, [_P, _P, _U64, _U8, _U32, _U32, _I, _MP]),
    "hkhip_free": (None, [_P, _MP]),
    "hkhip_dequantize": (_I, [_P, _MP, _U32, _U32, _P]),
    "hkhip_qact": (_I, [_P, _P, _U32, _U32, _I, _P]),
    "hkhip_act_export": (_I, [_P, _P, _U32, _U32, _I, _P]),
    "hkhip_matvec": (_I, [_P, _MP, _P, _P, _U32, _P, _I]),
    "hkhip_matvec_parts": (_I, [_P, _MP, _U32, _P, _P, _U32, _P, _P, _I]),
    "hkhip_matvec_parts_rmsnorm": (_I, [_P, _MP, _U32, _P, _P, ctypes.c_float, _U32, _P, _P, _I]),
    "hkhip_gemm": (_I, [_P, _MP, _P, _P, _U32, _P, _I]),
    "hkhip_mm": (_I, [_P, _MP, _P, _P, _U32, _P, _I]),
    "hkhip_mm_noalloc": (_I, [_P, _MP, _P, _P, _U32, _P, _I]),
    "hkhip_gemm_host": (_I, [_U8, _P, _P, _P, _P, _U64, _U64, _U64]),
    "hkhip_net_create": (_I, [_P, ctypes.POINTER(NetConfig), ctypes.POINTER(_P)]),
    "hkhip_net_create_opts": (_I, [_P, ctypes.POINTER(NetConfig), ctypes.POINTER(NetOptions), ctypes.POINTER(_P)]),
    "hkhip_net_forward_items": (_I, [_P, _P, _U32]),
    "hkhip_net_forward_partial": (_I, [_P, _P, _U32, _P]),
    "hkhip_net_logits_rows": (_I, [_P, _P, _U32, _P]),
    "hkhip_net_logits_view": (_I, [_P, _P, _U32, _P]),
    "hkhip_net_release": (None, [_P, _U64]),
    "hkhip_net_max_rows": (_U32, [_P]),
    "hkhip_net_layer_count": (_U32, [_P]),
    "hkhip_net_is_partial": (_I, [_P]),
    "hkhip_net_bytes_needed": (_U64, [ctypes.POINTER(NetConfig), ctypes.POINTER(NetOptions), ctypes.POINTER(NetLayer),
                                      NetTensor, NetTensor, NetTensor]),
    "hkhip_net_layer_bytes": (_U64, [ctypes.POINTER(NetConfig), ctypes.POINTER(NetLayer)]),
    "hkhip_net_device_bytes": (_U64, [_P]),
    "hkhip_net_destroy": (None, [_P]),
    "hkhip_net_load_layer": (_I, [_P, _U32, ctypes.POINTER(NetLayer)]),
    "hkhip_net_load_io": (_I, [_P, NetTensor, NetTensor, NetTensor]),
    "hkhip_net_forward": (_I, [_P, _P, _U32, _U32]),
    "hkhip_net_logits": (_I, [_P, _P]),
    "hkhip_net_logits_dev": (_P, [_P]),
    "hkhip_gemv_q8_0": (_I, [_P, _P, _P, _P, _U64, _U64]),
    "hkhip_gemv_q4_0": (_I, [_P, _P, _P, _P, _U64, _U64]),
    "hkhip_gemv_q4_k": (_I, [_P, _P, _P, _P, _U64, _U64]),
    "hkhip_gemv_q6_k": (_I, [_P, _P, _P, _P, _U64, _U64]),
    "hkhip_gemv_iq4_nl": (_I, [_P, _P, _P, _P, _U64, _U64]),
}

_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """Loads libhkhip.so, raising if it was not built (no silent fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python hk_amd/build.py` "
                               "(or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc < 0:
        msg = lib().hkhip_last_error()
        raise HipError(rc, msg.decode() if msg else "")
