"""NumPy restatement of the prefill GEMM's offline weight prepack (test
infrastructure only: ``tests/`` import it, the product never does).

The layout has no counterpart in the reference: it is this build's own
format for ``xrmm_prepack_weights`` (the "prepare = upload / prepack" step of
the reference's Operator lifecycle, kernels/_shared/extended/vulkan.cpp:119).
The codes stay the reference's (complex_kernel.glsl:80, low nibble first along
K); only their positions change:

* K-step-major: ``packed[s, n, :]`` holds the 32 bytes of codes
  ``64 s .. 64 s + 63`` of column ``n`` (two 16-byte halves of 32 codes; a
  half past the column's last 32-code chunk is zero);
* inside each little-endian 32-bit word, the eight codes ``c0 .. c7`` of
  eight consecutive k sit in nibble slots ``c0 c2 c4 c6 c1 c3 c5 c7``.

Pinned in ``tests/test_oracle.py`` by decoding the layout back with the GEMM's
own pair rule (slots 0/4, 1/5, 2/6, 3/7 give k order) and comparing with
``oracle.unpack_codes``, which is pinned independently.
"""
from __future__ import annotations

import numpy as np


def packed_bytes(N: int, K: int, block_size: int, bits: int = 4) -> int:
    kb = (K + block_size - 1) // block_size
    Kp = kb * block_size
    if bits != 4 or N <= 0 or Kp <= 0 or Kp % 32:
        return 0
    return (Kp + 63) // 64 * N * 32


def _squeeze(b: np.ndarray) -> np.ndarray:
    """Low nibbles of the four bytes of each word -> one 16-bit value."""
    t = (b | (b >> np.uint32(4))) & np.uint32(0x00FF00FF)
    return (t & np.uint32(0xFF)) | ((t >> np.uint32(8)) & np.uint32(0xFF00))


def prepack_q4(B: np.ndarray, K: int, block_size: int) -> np.ndarray:
    """B ``[N, kb, block_size // 2]`` uint8 -> flat uint8 prepacked layout."""
    B = np.ascontiguousarray(B, dtype=np.uint8)
    N, kb, blob = B.shape
    Kp = kb * block_size
    nbytes = packed_bytes(N, K, block_size)
    if nbytes == 0:
        raise ValueError("no prepacked layout for this geometry")
    ksteps = (Kp + 63) // 64
    rows = np.zeros((N, ksteps * 32), dtype=np.uint8)
    rows[:, : Kp // 2] = B.reshape(N, kb * blob)
    words = rows.view("<u4")
    lo = words & np.uint32(0x0F0F0F0F)
    hi = (words >> np.uint32(4)) & np.uint32(0x0F0F0F0F)
    packed_words = (_squeeze(lo) | (_squeeze(hi) << np.uint32(16))).astype("<u4")
    return np.ascontiguousarray(packed_words.view(np.uint8).reshape(N, ksteps, 32).transpose(1, 0, 2)).reshape(-1)
