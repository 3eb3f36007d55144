"""NumPy oracle for com.microsoft.GatherBlockQuantized (opcode 1031) and
com.microsoft.MatMulBnb4 (opcode 1026) (test infrastructure only).

This module is the oracle, test infrastructure and never the product: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` may import it.

It restates, on the CPU, the arithmetic of xrGPU's serial Vulkan shader:

* ``gatherQuant`` kernels/_shared/extended/shaders/complex_kernel.glsl:85 —
  for each index, the selected row's codes (low-first within a byte) minus the
  zero point (packed low-first per block, default 2^(bits-1)) times the
  block's float32 scale, rounded once in float32; an index outside
  [0, rows) fails the run with code 55 and leaves its output row zero
  (zero-filled outputs, complex_kernel.glsl:197; the host turns the code into
  "GPU operator contract validation failed: code 55", vulkan.cpp:115).
  Indices read through ``controlIndex`` (complex_kernel.glsl:31): int32 as is,
  int64 saturated to the int32 range. Planner: bits 4 or 8, block_size a
  power of two >= 16, gather_axis 0, quantize_axis 1, output
  [indices.shape[0], data.shape[1] * 8 / bits] in the scales' dtype
  (complex_plan.cpp:129).
* ``bnbWeight`` complex_kernel.glsl:82 and the 1026 branch of
  ``packedMatmul`` complex_kernel.glsl:83 — the flat weight index is
  ``n * K + k`` (transB, the default) or ``k * N + n``; two codes per byte with
  the even flat index in the HIGH nibble; the value is ``codebook[code] *
  absmax[flat / block_size]`` (NF4 for quant_type 1, the default, FP4 for 0);
  Y = A @ W summed in float32 and stored in A's dtype. Planner defaults
  block_size 32, quant_type 1, transB 1 (complex_plan.cpp:117-120).

Sums are float64, rounded once to the output dtype. Pins:
``tests/test_oracle_quant.py``.
"""
from __future__ import annotations

import numpy as np

GBQ_INDEX_ERROR = 55  # the shader's failure code for an out-of-range index

# bitsandbytes codebooks as the shader lists them (complex_kernel.glsl:82)
NF4 = np.array([-1.0, -0.6961928009986877, -0.5250730514526367, -0.3949174880981445, -0.28444138169288635,
                -0.18477343022823334, -0.09105003625154495, 0.0, 0.07958029955625534, 0.16093020141124725,
                0.24611230194568634, 0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
                0.7229568362236023, 1.0], dtype=np.float32)
FP4 = np.array([0.0, 0.0052083333333333, 0.6666666666666666, 1.0, 0.3333333333333333, 0.5, 0.1666666666666666, 0.25,
                -0.0, -0.0052083333333333, -0.6666666666666666, -1.0, -0.3333333333333333, -0.5,
                -0.1666666666666666, -0.25], dtype=np.float32)


class GatherIndexError(IndexError):
    """An index outside [0, rows): the reference fails the run with code 55."""


def control_index(indices) -> np.ndarray:
    """``controlIndex``: int32 indices as is, int64 saturated to int32."""
    idx = np.asarray(indices)
    if idx.dtype == np.int64:
        return np.clip(idx, -(2 ** 31), 2 ** 31 - 1).astype(np.int64)
    return idx.astype(np.int32).astype(np.int64)


def gather_block_quantized(data, indices, scales, zero_points=None, *, bits: int = 4, block_size: int = 128,
                           strict: bool = True):
    """GatherBlockQuantized output (float32, or the scales' dtype).

    With ``strict`` an out-of-range index raises ``GatherIndexError``;
    otherwise the output comes back with those rows zero, as the reference
    leaves them before failing the run.
    """
    data = np.asarray(data, np.uint8)
    sc = np.asarray(scales)
    rows, packed_cols = data.shape
    width = packed_cols * (8 // bits)
    blocks = (width + block_size - 1) // block_size
    idx = control_index(indices).reshape(-1)
    out = np.zeros((idx.size, width), np.float32)
    bad = (idx < 0) | (idx >= rows)
    if strict and bad.any():
        raise GatherIndexError(f"code {GBQ_INDEX_ERROR}")
    j = np.arange(width)
    shift = (j * bits) % 8
    mask = (1 << bits) - 1
    blk = j // block_size
    sc32 = sc.astype(np.float32).reshape(rows, blocks)
    for o, r in enumerate(idx):
        if bad[o]:
            continue
        q = (data[r, (j * bits) // 8].astype(np.uint32) >> shift) & mask
        if zero_points is not None:
            zrow = np.asarray(zero_points, np.uint8).reshape(rows, -1)[r]
            z = (zrow[(blk * bits) // 8].astype(np.uint32) >> ((blk * bits) % 8)) & mask
        else:
            z = np.full(width, 1 << (bits - 1), np.uint32)
        out[o] = (q.astype(np.float32) - z.astype(np.float32)) * sc32[r, blk]
    return out.astype(sc.dtype) if sc.dtype == np.float16 else out


def bnb_codes(b, count: int) -> np.ndarray:
    """Codes of flat indices 0..count-1: the even index in the high nibble."""
    b = np.asarray(b, np.uint8).reshape(-1)
    i = np.arange(count)
    byte = b[i // 2].astype(np.uint8)
    return np.where(i % 2 == 0, byte >> 4, byte & 15).astype(np.int64)


def bnb_weights(b, absmax, K: int, N: int, block_size: int, quant_type: int = 1, trans_b: int = 1) -> np.ndarray:
    """``bnbWeight`` for every (k, n): float32 [K, N]."""
    book = NF4 if quant_type == 1 else FP4
    am = np.asarray(absmax).astype(np.float32).reshape(-1)
    k = np.arange(K)[:, None]
    n = np.arange(N)[None, :]
    flat = n * K + k if trans_b else k * N + n
    codes = bnb_codes(b, K * N)[flat]
    return (book[codes] * am[flat // block_size]).astype(np.float32)


def matmul_bnb4(a, b, absmax, *, K: int, N: int, block_size: int = 32, quant_type: int = 1, trans_b: int = 1,
                out_dtype=None):
    """Y = A @ W (float64 sums, one rounding to A's dtype)."""
    a = np.asarray(a)
    W = bnb_weights(b, absmax, K, N, block_size, quant_type, trans_b).astype(np.float64)
    y = a.reshape(-1, K).astype(np.float64) @ W
    return y.reshape(*a.shape[:-1], N).astype(out_dtype or a.dtype)
