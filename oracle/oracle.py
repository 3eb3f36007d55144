"""NumPy oracle for the MatMulNBits operator family (test infrastructure only).

This module is the oracle, test infrastructure and never the product. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it. The product path (``xrgpu_amd``) never calls into it and fails
loudly when its HIP library is missing.

It restates, on the CPU, the arithmetic of xrGPU's serial Vulkan shader for
opcodes 1025 (MatMulNBits), 1027 (MatMulNBitsMlp) and 1028 (MatMulNBitsQkv):

* ``nbitWeight``   kernels/_shared/extended/shaders/complex_kernel.glsl:80
* ``packedInput``  kernels/_shared/extended/shaders/complex_kernel.glsl:81
* ``packedMatmul`` kernels/_shared/extended/shaders/complex_kernel.glsl:83
* ``fused``/``logistic`` complex_kernel.glsl:39-47 (activation kinds from
  ``activation_lower`` kernels/_shared/extended/complex_plan.cpp:55)
* planner defaults (block_size 32, bits 4, eps 1e-5 / 1e-6 for Qkv, activation
  silu) kernels/_shared/extended/complex_plan.cpp:118
* binary16 storage: IEEE round-to-nearest-even, which
  kernels/_shared/shaders/half.glsl:17-45 implements and which the reference
  proves equal to ``numpy.astype(float16)`` (tests/test_native_half.py:43-84).

Accumulation is done in float64 and rounded once to the output dtype; the
reference accumulates serially in float32 and also rounds once. Dequantized
weights follow the reference exactly in float32: ``(float(code) - z) * scale``.

Extensions beyond the reference contract (declared, not reference behaviour):

* packed uint8 zero points in the ONNX Runtime layout
  ``[N, ceil(k_blocks * bits / 8)]``, low-first (the reference only accepts
  float zero points, contract.json T3 = {float32, float16});
* zero points for the Qkv/Mlp projections (the reference passes NONE there,
  complex_kernel.glsl:83).

Parity pins for every function are listed in the module-level ``PINS`` table;
each entry names the test that pins it.
"""
from __future__ import annotations

import math

import numpy as np

ZP_NONE = "none"
ZP_FLOAT = "float"
ZP_PACKED = "packed"

# function -> the checks that pin it (tests/test_oracle.py)
PINS = {
    "unpack_codes": "brute force over all 256 bytes x bits {2,4,8}; Qkv KAT bytes 152/168/184",
    "unpack_packed_zero_points": "brute force nibble/crumb order; packed == float-zp invariant",
    "dequantize": "block-512 exact fixture (Y=128); closed form (code-z)*scale exact in fp32",
    "matmul_nbits": "block-512 exact fixture; empty-M fixtures; f16 cancellation fixtures (exact 0); brute-force loop on tiny shapes",
    "matmul_nbits_mlp": "Mlp pinned_plain_gb_ub / pinned_norm_nogb_noub / pinned_skipsum_gb_ub explicit outputs",
    "matmul_nbits_qkv": "Qkv KAT (complex_reference.py:251-272); Qkv == 3 x MatMulNBits on normalised input",
    "fused_activation": "silu fixtures (Mlp pinned); closed forms relu/sigmoid/tanh/identity; gelu: "
                        "x*Phi(x) at +-1, gelu(x)-gelu(-x)=x, the shader's own A&S 7.1.26 erf within 2e-7, "
                        "apart from the tanh form, serial erff order",
}

ACTIVATIONS = {
    # complex_plan.cpp:55 activation_lower
    "none": 0, "": 0, "identity": 0, "relu": 1, "silu": 2, "swish": 2,
    "gelu": 3, "tanh": 4, "sigmoid": 5, "swiglu": 6,
}


def k_blocks(K: int, block_size: int) -> int:
    """``blocks=(K+block-1)/block`` (complex_kernel.glsl:80)."""
    return (K + block_size - 1) // block_size


def blob_bytes(block_size: int, bits: int) -> int:
    """``blockBytes=(block*bits+7)/8`` (complex_kernel.glsl:80)."""
    return (block_size * bits + 7) // 8


def packed_zp_bytes(kb: int, bits: int) -> int:
    """Bytes per row of ORT-layout packed zero points: ``ceil(kb*bits/8)``."""
    return (kb * bits + 7) // 8


def unpack_codes(B: np.ndarray, K: int, bits: int, block_size: int) -> np.ndarray:
    """Integer codes ``q[n, k]`` for ``k < K`` (complex_kernel.glsl:80).

    ``element = k % block``; the byte is ``B[n, k // block, element*bits // 8]``
    and the code is ``(byte >> ((element*bits) % 8)) & (2**bits - 1)``:
    codes are packed low-first along K. Codes at ``k >= K`` inside the last
    block are padding and are never read.
    """
    B = np.asarray(B, dtype=np.uint8)
    N = B.shape[0]
    k = np.arange(K, dtype=np.int64)
    element = k % block_size
    block = k // block_size
    byte = (element * bits) // 8
    shift = ((element * bits) % 8).astype(np.uint8)
    mask = np.uint8((1 << bits) - 1)
    if N == 0 or K == 0:
        return np.zeros((N, K), dtype=np.uint8)
    return (B[:, block, byte] >> shift[None, :]) & mask


def unpack_packed_zero_points(zp: np.ndarray, kb: int, bits: int) -> np.ndarray:
    """Zero points from the ONNX Runtime packed-uint8 layout (extension).

    ``z[n, b] = (zp[n, (b*bits)//8] >> ((b*bits) % 8)) & (2**bits - 1)``,
    low-first along the block axis, the same packing rule as B's codes.
    """
    zp = np.asarray(zp, dtype=np.uint8)
    b = np.arange(kb, dtype=np.int64)
    byte = (b * bits) // 8
    shift = ((b * bits) % 8).astype(np.uint8)
    mask = np.uint8((1 << bits) - 1)
    if zp.shape[0] == 0 or kb == 0:
        return np.zeros((zp.shape[0], kb), dtype=np.uint8)
    return (zp[:, byte] >> shift[None, :]) & mask


def zero_point_matrix(zero_points, N: int, kb: int, bits: int, kind: str) -> np.ndarray:
    """Float32 ``z[n, b]``.

    Absent: ``2**(bits-1)`` (complex_kernel.glsl:80, ``float(1u<<(bits-1u))``).
    Float: the element widened to float32. Packed: see
    :func:`unpack_packed_zero_points`.
    """
    if kind == ZP_NONE or zero_points is None:
        return np.full((N, kb), float(1 << (bits - 1)), dtype=np.float32)
    if kind == ZP_FLOAT:
        return np.asarray(zero_points).astype(np.float32).reshape(N, kb)
    if kind == ZP_PACKED:
        return unpack_packed_zero_points(zero_points, kb, bits).astype(np.float32)
    raise ValueError("unknown zero-point kind: " + str(kind))


def zero_point_kind(zero_points) -> str:
    if zero_points is None:
        return ZP_NONE
    return ZP_PACKED if np.asarray(zero_points).dtype == np.uint8 else ZP_FLOAT


def dequantize(B, scales, zero_points, K: int, bits: int, block_size: int,
               zp_kind: str | None = None, stage: str = "f32") -> np.ndarray:
    """Dequantized ``W[n, k]`` (complex_kernel.glsl:80).

    ``stage="f32"`` is the reference value: ``(float32(code) - z) * scale``
    evaluated in float32 (one rounding per operation, as the shader does).
    ``stage="f16"`` is that float32 value rounded once to binary16 (RNE): the
    value an fp16 MFMA path stages into registers/LDS.
    """
    B = np.asarray(B, dtype=np.uint8)
    N = B.shape[0]
    kb = k_blocks(K, block_size)
    if zp_kind is None:
        zp_kind = zero_point_kind(zero_points)
    q = unpack_codes(B, K, bits, block_size).astype(np.float32)
    z = zero_point_matrix(zero_points, N, kb, bits, zp_kind)
    s = np.asarray(scales).astype(np.float32).reshape(N, kb)
    blk = np.arange(K) // block_size
    with np.errstate(all="ignore"):
        w = (q - z[:, blk]) * s[:, blk]
    w = w.astype(np.float32)
    if stage == "f32":
        return w
    if stage == "f16":
        with np.errstate(all="ignore"):
            return w.astype(np.float16)
    raise ValueError("stage must be f32 or f16")


def _round_to(x64: np.ndarray, dtype) -> np.ndarray:
    """One rounding from float64 to the storage dtype (RNE; half.glsl:17-45)."""
    with np.errstate(all="ignore"):
        # float64 -> float32 -> float16 could double-round; go through float32
        # only when the target is float32. numpy's float64->float16 cast is a
        # single correctly rounded conversion.
        return x64.astype(dtype)


def _rows(A: np.ndarray, K: int) -> np.ndarray:
    """``rows = size(A)/K`` (complex_kernel.glsl:83): leading axes fold."""
    A = np.asarray(A)
    return A.reshape(-1, K) if A.size else A.reshape(0, K)


def logistic(x):
    """``x>=0 ? 1/(1+e^-x) : e^x/(1+e^x)`` (complex_kernel.glsl:39)."""
    x = np.asarray(x, dtype=np.float64)
    with np.errstate(over="ignore"):
        e = np.exp(-np.abs(x))
    return np.where(x >= 0, 1.0 / (1.0 + e), e / (1.0 + e))


def fused_activation(x, kind: int):
    """``fused(x, kind)`` (complex_kernel.glsl:41-47) for opcode 1027."""
    x = np.asarray(x, dtype=np.float64)
    if kind == 1:
        return np.maximum(x, 0.0)
    if kind == 2:
        return x * logistic(x)
    if kind == 3:
        # opcode 1027 uses the erf form (complex_kernel.glsl:42-43)
        from scipy.special import erf
        return 0.5 * x * (1.0 + erf(x * 0.7071067811865475))
    if kind == 4:
        return np.tanh(x)
    if kind == 5:
        return logistic(x)
    return x


def normalized_input(A, K: int, skip=None, norm_scale=None, epsilon: float = 1e-5):
    """``packedInput`` with ``normalized=true`` (complex_kernel.glsl:81).

    ``r = A + skip`` (float32 add); if ``norm_scale`` is present,
    ``x = r * inversesqrt(sum(r^2)/K + eps) * gamma[k]``. ``eps`` is stored as
    float32 by the planner (complex_plan.cpp:118, ``fword(float(...))``).
    Returns ``(x64, r32)``: the float64 normalised input and the float32
    residual sum that the optional ``residualT`` output stores.
    """
    a = _rows(A, K).astype(np.float32)
    r = a if skip is None else (a + _rows(skip, K).astype(np.float32)).astype(np.float32)
    x = r.astype(np.float64)
    if norm_scale is not None:
        eps = float(np.float32(epsilon))
        ms = np.mean(x * x, axis=1, keepdims=True) if K else np.zeros((x.shape[0], 1))
        g = np.asarray(norm_scale).astype(np.float32).astype(np.float64).reshape(1, K)
        x = x / np.sqrt(ms + eps) * g
    return x, r


def matmul_nbits(A, B, scales, zero_points=None, bias=None, *, K: int, N: int,
                 bits: int = 4, block_size: int = 32, zp_kind: str | None = None,
                 out_dtype=None) -> np.ndarray:
    """com.microsoft.MatMulNBits, opcode 1025 (complex_kernel.glsl:83).

    ``Y[..., n] = sum_k A[..., k] * W[n, k] + bias[n]``, accumulated here in
    float64 over the reference's float32 ``W`` and rounded once to A's dtype.
    Output shape ``A.shape[:-1] + [N]`` (complex_plan.cpp:119).
    """
    A = np.asarray(A)
    out_dtype = out_dtype or A.dtype
    x = _rows(A, K).astype(np.float64)
    W = dequantize(B, scales, zero_points, K, bits, block_size, zp_kind).astype(np.float64)
    y = x @ W.T if x.shape[0] else np.zeros((0, N))
    if bias is not None:
        y = y + np.asarray(bias).astype(np.float32).astype(np.float64)[None, :]
    return _round_to(y, out_dtype).reshape(tuple(A.shape[:-1]) + (N,))


def matmul_nbits_qkv(A, q_B, q_scales, k_B, k_scales, v_B, v_scales, *, K: int, Nq: int,
                     Nkv: int, norm_scale, skip=None, bits: int = 4, block_size: int = 32,
                     epsilon: float = 1e-6, q_zero_points=None, k_zero_points=None,
                     v_zero_points=None, out_dtype=None):
    """com.microsoft.MatMulNBitsQkv, opcode 1028 (complex_kernel.glsl:81,83).

    ``x = RMSNorm(A + skip) * gamma``; Q/K/V are three projections of the same
    x with their own packed weights (B/scales slots 3/4, 5/6, 7/8). Returns
    ``(Q, K, V, residual)``; residual is ``A + skip`` rounded to A's dtype.
    Zero points are an extension (the reference uses the implicit midpoint).
    """
    A = np.asarray(A)
    out_dtype = out_dtype or A.dtype
    x, r = normalized_input(A, K, skip, norm_scale, epsilon)
    lead = tuple(A.shape[:-1])
    outs = []
    for Bm, S, Z, n in ((q_B, q_scales, q_zero_points, Nq), (k_B, k_scales, k_zero_points, Nkv),
                        (v_B, v_scales, v_zero_points, Nkv)):
        W = dequantize(Bm, S, Z, K, bits, block_size).astype(np.float64)
        y = x @ W.T if x.shape[0] else np.zeros((0, n))
        outs.append(_round_to(y, out_dtype).reshape(lead + (n,)))
    outs.append(_round_to(r.astype(np.float64), out_dtype).reshape(A.shape))
    return tuple(outs)


def matmul_nbits_mlp(A, gate_B, gate_scales, up_B, up_scales, *, K: int, N: int,
                     skip=None, norm_scale=None, gate_bias=None, up_bias=None,
                     bits: int = 4, block_size: int = 32, epsilon: float = 1e-5,
                     activation: str = "silu", gate_zero_points=None, up_zero_points=None,
                     out_dtype=None):
    """com.microsoft.MatMulNBitsMlp, opcode 1027 (complex_kernel.glsl:39-47,81,83).

    ``x = A + skip`` (normalised by RMSNorm * gamma when ``norm_scale`` is
    given); ``Y = fused(x@Wg^T + gate_bias, act) * (x@Wu^T + up_bias)``.
    Returns ``(Y, residual)``.
    """
    A = np.asarray(A)
    out_dtype = out_dtype or A.dtype
    kind = ACTIVATIONS[activation]
    x, r = normalized_input(A, K, skip, norm_scale, epsilon)
    lead = tuple(A.shape[:-1])
    Wg = dequantize(gate_B, gate_scales, gate_zero_points, K, bits, block_size).astype(np.float64)
    Wu = dequantize(up_B, up_scales, up_zero_points, K, bits, block_size).astype(np.float64)
    g = x @ Wg.T if x.shape[0] else np.zeros((0, N))
    u = x @ Wu.T if x.shape[0] else np.zeros((0, N))
    if gate_bias is not None:
        g = g + np.asarray(gate_bias).astype(np.float32).astype(np.float64)[None, :]
    if up_bias is not None:
        u = u + np.asarray(up_bias).astype(np.float32).astype(np.float64)[None, :]
    y = fused_activation(g, kind) * u
    return (_round_to(y, out_dtype).reshape(lead + (N,)),
            _round_to(r.astype(np.float64), out_dtype).reshape(A.shape))


def tolerance_ok(actual, expected, dtype) -> tuple[bool, float, float]:
    """The parity bar: ``max|d| <= 1e-2*max|Y_ref|`` (fp16), ``1e-5*max|Y_ref|`` (fp32).

    Returns ``(ok, max_abs_err, limit)``. Non-finite values must match exactly:
    +-Inf with the same sign, NaN where the expectation is NaN (the
    ``allowNaN`` policy of kernels/_shared/verify_upstream.py:130-142).
    """
    a = np.asarray(actual).astype(np.float64)
    e = np.asarray(expected).astype(np.float64)
    if a.shape != e.shape:
        return False, math.inf, 0.0
    if a.size == 0:
        return True, 0.0, 0.0
    fin = np.isfinite(e)
    if not np.array_equal(np.isfinite(a), fin):
        return False, math.inf, 0.0
    if not np.all((a == e) | fin | (np.isnan(a) & np.isnan(e))):
        return False, math.inf, 0.0
    rel = 1e-2 if np.dtype(dtype) == np.float16 else 1e-5
    ref = float(np.max(np.abs(e[fin]))) if fin.any() else 0.0
    err = float(np.max(np.abs(a[fin] - e[fin]))) if fin.any() else 0.0
    limit = rel * ref
    return err <= limit, err, limit
