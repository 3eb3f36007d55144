"""ctypes wrapper of ``oracle_serial.c`` (test infrastructure only).

Gives the reference's own float32 serial summation order
(kernels/_shared/extended/shaders/complex_kernel.glsl:83) for small shapes, so
tests can check that the float64 NumPy oracle and the float32 serial order
agree far inside the parity tolerance.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_serial.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_i64 = ctypes.c_int64


def build() -> str:
    """Compile ``oracle_serial.c`` with the committed Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        lib.oracle_matmul_nbits.argtypes = [_f32p, _u8p, _f32p, ctypes.c_int, _f32p, _u8p, _f32p,
                                            _f32p, _i64, _i64, _i64, ctypes.c_int, _i64]
        lib.oracle_matmul_nbits.restype = None
        lib.oracle_matmul_nbits_mlp.argtypes = [_f32p, _f32p, _f32p, ctypes.c_float, _u8p, _f32p,
                                                _f32p, _u8p, _f32p, _f32p, ctypes.c_int, _f32p,
                                                _f32p, _f32p, _i64, _i64, _i64, ctypes.c_int, _i64]
        lib.oracle_matmul_nbits_mlp.restype = None
        lib.oracle_matmul_nbits_qkv.argtypes = [_f32p, _f32p, _f32p, ctypes.c_float,
                                                ctypes.POINTER(_u8p), ctypes.POINTER(_f32p),
                                                ctypes.c_int, ctypes.POINTER(_f32p),
                                                ctypes.POINTER(_u8p), _f32p, _f32p, _f32p, _f32p,
                                                _f32p, _i64, _i64, _i64, _i64, ctypes.c_int, _i64]
        lib.oracle_matmul_nbits_qkv.restype = None
        _lib = lib
    return _lib


def _f(x):
    if x is None:
        return None
    return np.ascontiguousarray(np.asarray(x).astype(np.float32))


def _p(x, t):
    return None if x is None else x.ctypes.data_as(t)


def matmul_nbits(A, B, scales, zero_points=None, bias=None, *, K, N, bits=4, block_size=32):
    """Serial float32 result of opcode 1025, before the output rounding."""
    lib = _load()
    a = _f(np.asarray(A).reshape(-1, K))
    M = a.shape[0]
    b = np.ascontiguousarray(B, dtype=np.uint8)
    s = _f(scales)
    zk, zf, zq = 0, None, None
    if zero_points is not None:
        z = np.asarray(zero_points)
        if z.dtype == np.uint8:
            zk, zq = 2, np.ascontiguousarray(z)
        else:
            zk, zf = 1, _f(z)
    bi = _f(bias)
    y = np.zeros((M, N), np.float32)
    lib.oracle_matmul_nbits(_p(a, _f32p), _p(b, _u8p), _p(s, _f32p), zk, _p(zf, _f32p),
                            _p(zq, _u8p), _p(bi, _f32p), _p(y, _f32p), M, K, N, bits, block_size)
    return y


def matmul_nbits_mlp(A, gate_B, gate_scales, up_B, up_scales, *, K, N, skip=None, norm_scale=None,
                     gate_bias=None, up_bias=None, bits=4, block_size=32, epsilon=1e-5, act=2):
    lib = _load()
    a = _f(np.asarray(A).reshape(-1, K))
    M = a.shape[0]
    sk = None if skip is None else _f(np.asarray(skip).reshape(-1, K))
    g = _f(norm_scale)
    y = np.zeros((M, N), np.float32)
    r = np.zeros((M, K), np.float32)
    x = np.zeros((M, K), np.float32)
    gb, ub = np.ascontiguousarray(gate_B, np.uint8), np.ascontiguousarray(up_B, np.uint8)
    gs, us = _f(gate_scales), _f(up_scales)
    gbi, ubi = _f(gate_bias), _f(up_bias)
    lib.oracle_matmul_nbits_mlp(_p(a, _f32p), _p(sk, _f32p), _p(g, _f32p), float(np.float32(epsilon)),
                                _p(gb, _u8p), _p(gs, _f32p), _p(gbi, _f32p), _p(ub, _u8p),
                                _p(us, _f32p), _p(ubi, _f32p), act, _p(y, _f32p), _p(r, _f32p),
                                _p(x, _f32p), M, K, N, bits, block_size)
    return y, r


def matmul_nbits_qkv(A, Bs, Ss, *, K, Nq, Nkv, norm_scale, skip=None, zero_points=None, bits=4,
                     block_size=32, epsilon=1e-6):
    lib = _load()
    a = _f(np.asarray(A).reshape(-1, K))
    M = a.shape[0]
    sk = None if skip is None else _f(np.asarray(skip).reshape(-1, K))
    g = _f(norm_scale)
    bs = [np.ascontiguousarray(b, np.uint8) for b in Bs]
    ss = [_f(s) for s in Ss]
    barr = (_u8p * 3)(*[_p(b, _u8p) for b in bs])
    sarr = (_f32p * 3)(*[_p(s, _f32p) for s in ss])
    zk, zfa, zqa, keep = 0, None, None, []
    if zero_points is not None:
        zs = [np.asarray(z) for z in zero_points]
        if zs[0].dtype == np.uint8:
            zk = 2
            keep = [np.ascontiguousarray(z) for z in zs]
            zqa = (_u8p * 3)(*[_p(z, _u8p) for z in keep])
        else:
            zk = 1
            keep = [_f(z) for z in zs]
            zfa = (_f32p * 3)(*[_p(z, _f32p) for z in keep])
    q = np.zeros((M, Nq), np.float32)
    k = np.zeros((M, Nkv), np.float32)
    v = np.zeros((M, Nkv), np.float32)
    r = np.zeros((M, K), np.float32)
    x = np.zeros((M, K), np.float32)
    lib.oracle_matmul_nbits_qkv(_p(a, _f32p), _p(sk, _f32p), _p(g, _f32p), float(np.float32(epsilon)),
                                barr, sarr, zk, zfa, zqa, _p(q, _f32p), _p(k, _f32p), _p(v, _f32p),
                                _p(r, _f32p), _p(x, _f32p), M, K, Nq, Nkv, bits, block_size)
    return q, k, v, r
