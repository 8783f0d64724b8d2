"""ctypes binding of libdirktensor_amd.so (the C ABI declared in include/dirktensor_amd.h).

Loading fails loudly when the shared library is missing: there is no CPU
fallback for any entry point.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libdirktensor_amd.so"

DT_OK = 0
DT_ERR_INVALID_ARG = -1
DT_ERR_UNSUPPORTED = -2
DT_ERR_HIP = -3
DT_ERR_BLAS = -4
DT_ERR_NOT_IMPLEMENTED = -5
DT_ERR_IO = -6

DT_FP32_EXACT = 0
DT_BF16 = 1
DT_MEM_DEVICE = 0
DT_MEM_HOST = 1

DT_OPT_QKV_FUSED = 1
DT_QKV_GEMM = 0
DT_QKV_FUSED = 1
DT_QKV_AUTO = 2
DT_OPT_GEMM_TUNE = 2
DT_OPT_BWD_DQ = 3
DT_OPT_QKV_SPIN_LIMIT = 4
DT_OPT_SIDE_STREAM = 5
DT_BWD_DQ_RECOMPUTE = 0
DT_BWD_DQ_FROM_DS = 1
DT_BWD_DQ_AUTO = 2

HEAD_DIM = 128
MAX_SEQ_LEN = 8192
D_MODEL = 2048
N_HEADS = 16

_c_int = ctypes.c_int
_vp = ctypes.c_void_p
_fp = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)

# name -> (restype, argtypes); must match include/dirktensor_amd.h
SIGNATURES = {
    "dt_last_error": (ctypes.c_char_p, []),
    "dt_version": (_c_int, []),
    "dt_ctx_create": (_c_int, [_c_int, ctypes.POINTER(_vp)]),
    "dt_ctx_destroy": (_c_int, [_vp]),
    "dt_ctx_set_option": (_c_int, [_vp, _c_int, _c_int]),
    "dt_ctx_check": (_c_int, [_vp]),
    "dt_rope_table_init": (_c_int, [_vp, ctypes.c_float, _c_int]),
    "dt_flash_attn_fwd": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int,
                                   ctypes.c_float, _c_int, _vp, _c_int, _c_int, _vp]),
    "dt_flash_attn_bwd": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int,
                                   _c_int, ctypes.c_float, _c_int, _c_int, _c_int, _vp]),
    "dt_flash_attn_bwd_noalloc": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int,
                                           _c_int, _c_int, ctypes.c_float, _c_int, _c_int, _vp]),
    "dt_qk_norm_rope_fwd": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int,
                                     _c_int, _c_int, _c_int, _c_int, _vp]),
    "dt_attn_layer_create": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, ctypes.POINTER(_vp)]),
    "dt_attn_layer_load": (_c_int, [_vp, ctypes.c_char_p, ctypes.c_uint, ctypes.POINTER(_vp)]),
    "dt_attn_layer_destroy": (_c_int, [_vp]),
    "dt_attn_layer_fwd": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _vp, _c_int, _c_int, _c_int, _vp]),
    "dt_attn_layer_bwd": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _vp]),
    "dt_attn_layer_step": (_c_int, [_vp, ctypes.c_float, _vp]),
    "dt_attn_layer_zero_grad": (_c_int, [_vp, _vp]),
    "dt_attn_layer_get_weights": (_c_int, [_vp] * 7 + [_c_int, _vp]),
    "dt_attn_layer_get_grads": (_c_int, [_vp] * 7 + [_c_int, _vp]),
    "dt_model_create": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _c_int, ctypes.POINTER(_vp)]),
    "dt_model_load": (_c_int, [_vp, ctypes.c_char_p, _c_int, ctypes.POINTER(_vp)]),
    "dt_model_destroy": (_c_int, [_vp]),
    "dt_model_set_param": (_c_int, [_vp, ctypes.c_char_p, _vp, ctypes.c_int64, _c_int]),
    "dt_model_get_param": (_c_int, [_vp, ctypes.c_char_p, _vp, ctypes.c_int64, _c_int, _c_int, _vp]),
    "dt_model_fwd": (_c_int, [_vp, _vp, _c_int, _c_int, _vp, _c_int, _c_int, _c_int, _vp]),
    "dt_model_bwd": (_c_int, [_vp, _vp, _c_int, _vp]),
    "dt_model_step": (_c_int, [_vp, ctypes.c_float, _vp]),
    "dt_model_zero_grad": (_c_int, [_vp, _vp]),
    "dt_ce_loss": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _c_int, _vp]),
}

_lib = None


class DTError(RuntimeError):
    """A C-ABI call returned a negative status; ``code`` holds it."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def lib() -> ctypes.CDLL:
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m dirktensor_amd.build_ext` "
                "(the attention path has no CPU fallback)")
        l = ctypes.CDLL(os.fspath(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def check(rc: int) -> None:
    if rc != DT_OK:
        msg = lib().dt_last_error().decode(errors="replace")
        raise DTError(rc, msg)


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))
