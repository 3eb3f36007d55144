"""ctypes binding of libxrmm.so (the C ABI declared in include/xrmm.h).

Loading fails loudly when the library has not been built: there is no CPU
fallback for any operator in this package.
"""
from __future__ import annotations

import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
# XRMM_LIB_PATH selects another build of the same ABI (the host-sanitizer
# build of xrgpu_amd/build_sanitized.py)
LIB_PATH = os.environ.get("XRMM_LIB_PATH") or os.path.join(HERE, "lib", "libxrmm.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "xrmm.h")

XRMM_OK, XRMM_EINVAL, XRMM_EDEVICE = 0, 1, 2
F32, F16, I32, U32, I16, I8, U8, I64, BOOL, UNSPECIFIED = range(10)
ACT = {"none": 0, "": 0, "identity": 0, "relu": 1, "silu": 2, "swish": 2, "gelu": 3,
       "tanh": 4, "sigmoid": 5, "swiglu": 6}

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float

_lib = None


class XrmmError(RuntimeError):
    """Device-side failure (the reference's std::runtime_error class)."""


class XrmmInvalid(ValueError):
    """Contract / geometry failure (the reference's std::invalid_argument class)."""


def declared_symbols() -> list[str]:
    """Function names declared in include/xrmm.h."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(xrmm_[a-z0-9_]+)\s*\(", text)))


def _sig(lib):
    def s(name, res, *args):
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = list(args)

    s("xrmm_last_error", ctypes.c_char_p)
    s("xrmm_version", ctypes.c_char_p)
    s("xrmm_matmul_nbits", ctypes.c_int, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _i32, _i32, _i32, _vp)
    s("xrmm_matmul_nbits_qkv", ctypes.c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32,
      _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _i32, _f32, _i32, _vp)
    s("xrmm_matmul_nbits_mlp", ctypes.c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32,
      _vp, _vp, _i64, _i64, _i64, _i32, _i32, _f32, _i32, _i32, _vp)
    s("xrmm_matmul_nbits_qkv_ws", ctypes.c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32,
      _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _i32, _f32, _i32, _vp, _i64, _vp)
    s("xrmm_matmul_nbits_mlp_ws", ctypes.c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32,
      _vp, _vp, _i64, _i64, _i64, _i32, _i32, _f32, _i32, _i32, _vp, _i64, _vp)
    s("xrmm_matmul_nbits_fused_workspace_bytes", _i64, _i32, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32)
    s("xrmm_dequantize", ctypes.c_int, _vp, _vp, _vp, _i32, _vp, _i64, _i64, _i32, _i32, _i32, _i32, _vp)
    s("xrmm_select_kernel", ctypes.c_char_p, _i32, _i64, _i64, _i64, _i32, _i32, _i32, _i32)
    s("xrmm_qmoe_workspace_bytes", _i64, _i64, _i32, _i64, _i64)
    s("xrmm_qmoe", ctypes.c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i32, _i32,
      _i32, _i32, _i32, _f32, _f32, _f32, _i32, _vp)
    s("xrmm_qmoe_kernel", ctypes.c_char_p, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32)
    s("xrmm_gather_block_quantized", ctypes.c_int, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _i32,
      _vp)
    s("xrmm_matmul_bnb4", ctypes.c_int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _vp)
    s("xrmm_matmul_bnb4_kernel", ctypes.c_char_p, _i64, _i64, _i64, _i32, _i32, _i32, _i32)
    s("xrmm_matmul_nbits_int8a_workspace_bytes", _i64, _i64, _i64)
    s("xrmm_matmul_nbits_int8a", ctypes.c_int, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32,
      _i32, _i32, _vp)
    s("xrmm_matmul_nbits_int8a_noalloc", ctypes.c_int, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _i32,
      _i32, _i32, _vp)
    s("xrmm_stream_read", ctypes.c_int, _vp, ctypes.c_uint64, _vp, _i32, _vp)
    s("xrmm_stream_read_ex", ctypes.c_int, _vp, ctypes.c_uint64, _vp, _i32, _i32, _i32, _vp)
    s("xrmm_mfma_peak_operand_bytes", _i64)
    s("xrmm_mfma_peak_flops", _i64, _i32, _i32, _i32)
    s("xrmm_mfma_peak", ctypes.c_int, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp)
    s("xrmm_matmul_nbits_workspace_bytes", _i64, _i64, _i64, _i64, _i32, _i32, _i32)
    s("xrmm_matmul_nbits_ws", ctypes.c_int, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _i32, _i32, _i32,
      _vp, _i64, _vp)
    s("xrmm_prepacked_bytes", _i64, _i64, _i64, _i32, _i32)
    s("xrmm_prepack_weights", ctypes.c_int, _vp, _vp, _i64, _i64, _i32, _i32, _vp)
    s("xrmm_matmul_nbits_prepacked", ctypes.c_int, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _i32, _i32,
      _i32, _vp)


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"libxrmm.so is not built ({LIB_PATH}); run `python -m xrgpu_amd.build`. "
                "There is no CPU fallback.")
        lib_ = ctypes.CDLL(LIB_PATH)
        _sig(lib_)
        _lib = lib_
    return _lib


def last_error() -> str:
    return lib().xrmm_last_error().decode()


def check(rc: int) -> None:
    if rc == XRMM_OK:
        return
    msg = last_error()
    if rc == XRMM_EINVAL:
        raise XrmmInvalid(msg)
    raise XrmmError(msg)
