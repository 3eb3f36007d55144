"""NumPy oracle of the opt-in int8-activation MatMulNBits path (accuracy_level
4; test infrastructure only: ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` may import it).

This is NOT the reference's arithmetic. xrGPU's shader computes MatMulNBits
in float32 for every accuracy_level (kernels/_shared/extended/shaders/
complex_kernel.glsl:83; the planner, complex_plan.cpp:118, reads no
accuracy_level). The upstream WebGPU operator quantizes A for
accuracy_level 4 (upstream cases ``q4_dp4a_prefill_al4_*`` and
``ort_f16_accuracy_level4_*`` of kernels/_provenance/upstream/
com.microsoft.MatMulNBits/build/webgpu/test.json, tolerance 0.02-0.03, and
the manifest variant ``q4_dp4a_prefill``: "quantizes A per 128 elements
(max_abs/127)"). The upstream quantizer's source is not in the reference, so
its exact rounding is unknown; this oracle fixes one:

* per row and block of 128 activations: ``scale = float32(max|a|) / 127``
  (float32), ``q = rint(a / scale)`` (float32 division, round half to even,
  within [-127, 127]); a block of zeros has scale 0 and codes 0;
* ``Y[m, n] = sum over blocks of scale[m, b] * sum_k q[m, k] * W[n, k]`` with
  the reference's float32 ``W`` (``oracle.dequantize``), float64 sums, one
  rounding to A's dtype (+ bias).

Pins (``tests/test_oracle_int8a.py``): activations that are exact multiples
of their block's scale reproduce the float32 MatMulNBits result, and for any
input the difference from it stays within the quantization bound
``sum_k |W[n, k]| * scale[m, b(k)] / 2``.
"""
from __future__ import annotations

import numpy as np

from . import oracle as O

QBLOCK = 128


def quantize_activations(A, K: int):
    """int8 codes [M, K] and float32 scales [M, K / 128] of the rows of A."""
    x = np.asarray(A).reshape(-1, K).astype(np.float32)
    M = x.shape[0]
    blocks = x.reshape(M, K // QBLOCK, QBLOCK)
    amax = np.abs(blocks).max(axis=2) if M else np.zeros((0, K // QBLOCK), np.float32)
    scale = (amax.astype(np.float32) / np.float32(127)).astype(np.float32)
    safe = np.where(scale == 0, np.float32(1), scale)
    q = np.rint((blocks / safe[:, :, None]).astype(np.float32))
    q = np.where(scale[:, :, None] == 0, 0, np.clip(q, -127, 127)).astype(np.int8)
    return q.reshape(M, K), scale


def matmul_nbits_int8a(A, B, scales, zero_points=None, bias=None, *, K: int, N: int, bits: int = 4,
                       block_size: int = 32, zp_kind=None, out_dtype=None):
    A = np.asarray(A)
    out_dtype = out_dtype or A.dtype
    q, s = quantize_activations(A, K)
    W = O.dequantize(B, scales, zero_points, K, bits, block_size, zp_kind).astype(np.float64)
    M = q.shape[0]
    y = np.zeros((M, N))
    for b in range(K // QBLOCK):
        sl = slice(b * QBLOCK, (b + 1) * QBLOCK)
        y += s[:, b:b + 1].astype(np.float64) * (q[:, sl].astype(np.float64) @ W[:, sl].T)
    if bias is not None:
        y = y + np.asarray(bias).astype(np.float32).astype(np.float64)[None, :]
    return O._round_to(y, out_dtype).reshape(tuple(A.shape[:-1]) + (N,))


def quantization_bound(A, B, scales, zero_points=None, *, K: int, bits: int = 4, block_size: int = 32,
                       zp_kind=None) -> np.ndarray:
    """Largest |Y_int8a - Y_exact| the rounding of A can cause: [M, N]."""
    _, s = quantize_activations(A, K)
    W = np.abs(O.dequantize(B, scales, zero_points, K, bits, block_size, zp_kind).astype(np.float64))
    per_k = np.repeat(s.astype(np.float64), QBLOCK, axis=1) / 2
    return per_k @ W.T
