"""ctypes binding of libnq_hip.so (the C ABI declared in include/nq.h).

Loading fails loudly when the library is missing: there is no CPU fallback
anywhere in this package.
"""
from __future__ import annotations

import ctypes
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libnq_hip.so")

NQ_OK, NQ_BAD_SHAPE, NQ_BAD_ALIGN, NQ_HIP_ERROR, NQ_BAD_ARG, NQ_IO_ERROR = 0, 1, 2, 3, 4, 5
NQ_F32, NQ_F16 = 0, 1
NQ_PATH_AUTO, NQ_PATH_GEMV, NQ_PATH_MFMA, NQ_PATH_GENERIC = 0, 1, 2, 3

_P = ctypes.c_void_p
_I = ctypes.c_int64
_D = ctypes.c_int
_Z = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/nq.h one to one.
SIGNATURES = {
    "nq_version": (ctypes.c_char_p, []),
    "nq_status_name": (ctypes.c_char_p, [ctypes.c_int]),
    "nq_last_error": (ctypes.c_char_p, []),
    "nq_quantize_q8": (_D, [_P, _I, _I, _P, _P, _P]),
    "nq_quantize_q4g": (_D, [_P, _I, _I, _I, _P, _P, _D, _P]),
    "nq_dequantize_q8": (_D, [_P, _P, _I, _I, _P, _D, _P]),
    "nq_dequantize_q4g": (_D, [_P, _P, _D, _I, _I, _I, _P, _D, _P]),
    "nq_act_quant_i8": (_D, [_P, _D, _I, _I, _P, _P, _P]),
    "nq_act_quant_i8_heads": (_D, [_P, _D, _I, _I, _I, _P, _P, _P]),
    "nq_rmsnorm_quant_i8": (_D, [_P, _D, _P, ctypes.c_float, _I, _I, _P, _P, _P]),
    "nq_add_rmsnorm_quant_i8": (_D, [_P, _P, _D, _P, ctypes.c_float, _I, _I, _P, _P, _P, _P]),
    "nq_silu_mul_quant_i8": (_D, [_P, _P, _D, _I, _I, _I, _P, _P, _P]),
    "nq_linear_q8": (_D, [_P, _D, _P, _P, _P, _P, _D, _I, _I, _I, _P]),
    "nq_linear_q4g": (_D, [_P, _D, _P, _P, _D, _I, _P, _P, _D, _I, _I, _I, _P]),
    "nq_linear_wq_workspace_size": (_Z, [_I, _I, _I]),
    "nq_linear_q8_ws": (_D, [_P, _D, _P, _P, _P, _P, _D, _I, _I, _I, _P, _Z, _P]),
    "nq_linear_q4g_ws": (_D, [_P, _D, _P, _P, _D, _I, _P, _P, _D, _I, _I, _I, _P, _Z, _P]),
    "nq_linear_q8_ex": (_D, [_P, _D, _P, _P, _P, _P, _D, _I, _I, _I, _P, _Z, _D, _P]),
    "nq_linear_q4g_ex": (_D, [_P, _D, _P, _P, _D, _I, _P, _P, _D, _I, _I, _I, _P, _Z, _D, _P]),
    "nq_lm_head_argmax_q8_workspace_size": (_Z, [_I, _I, _I]),
    "nq_lm_head_argmax_q8": (_D, [_P, _D, _P, _P, _P, _P, _I, _I, _I, _P, _Z, _P]),
    "nq_linear_w8a8_workspace_size": (_Z, [_I, _I, _I]),
    "nq_linear_w8a8": (_D, [_P, _D, _P, _P, _P, _P, _D, _I, _I, _I, _P, _Z, ctypes.c_int, _P]),
    "nq_linear_w8a8_noalloc_max_scratch": (_Z, []),
    "nq_linear_w8a8_noalloc": (_D, [_P, _D, _P, _P, _P, _P, _D, _I, _I, _I, ctypes.c_int, _P]),
    "nq_gemm_w8a8_workspace_size": (_Z, [_I, _I, _I]),
    "nq_gemm_w8a8": (_D, [_P, _P, _P, _P, _P, _P, _D, _I, _I, _I, _P, _Z, ctypes.c_int, _P]),
    "nq_w8a8_acc_i32": (_D, [_P, _P, _P, _I, _I, _I, _P, _Z, ctypes.c_int, _P]),
    "nq_embedding_q8": (_D, [_P, _P, _I, _I, _P, _I, _P, _D, _P]),
    "nq_rope_qkv": (_D, [_P, _D, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P]),
    "nq_rmsnorm_f32": (_D, [_P, _P, _P, _P, ctypes.c_float, _I, _I, _P, _P]),
    "nq_silu_mul_f32": (_D, [_P, _P, _I, _I, _I, _P, _P]),
    "nq_attention_causal_f32": (_D, [_P, _P, _P, _I, _I, _I, _I, _P, _P]),
    "nq_nit_info": (_D, [ctypes.c_char_p, _P, _P, _P, ctypes.c_int32]),
    "nq_nit_load_f32": (_D, [ctypes.c_char_p, _P, _I, _P]),
    "nq_nit_load_q8": (_D, [ctypes.c_char_p, _P, _P, _I, _I, _P]),
    "nq_nit_load_q4g": (_D, [ctypes.c_char_p, _P, _P, _D, _I, _I, _I, _P]),
}


class NqError(RuntimeError):
    """A non-NQ_OK status from libnq_hip.so."""

    def __init__(self, status: int, name: str, message: str):
        super().__init__(f"{name}: {message}")
        self.status = status


class NqShapeError(NqError, ValueError):
    """NQ_BAD_SHAPE / NQ_BAD_ARG / NQ_BAD_ALIGN: the reference's std::invalid_argument."""


_lib = None


def load(path: str = LIB_PATH):
    """Load libnq_hip.so once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(
            f"{path} is missing: build it with `python -m nanoinfer_amd.build` "
            "(the quant path has no CPU fallback)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(status: int) -> None:
    """Raise the matching Python exception for a failed call."""
    if status == NQ_OK:
        return
    lib = load()
    name = lib.nq_status_name(status).decode()
    msg = lib.nq_last_error().decode()
    if status in (NQ_BAD_SHAPE, NQ_BAD_ARG, NQ_BAD_ALIGN):
        raise NqShapeError(status, name, msg)
    raise NqError(status, name, msg)
