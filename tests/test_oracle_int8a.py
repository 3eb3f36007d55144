"""Pins of the opt-in int8-activation oracle (oracle/int8a.py), CPU.

Not reference behaviour (the reference computes in float32 at every
accuracy_level), so it is pinned against the float32 MatMulNBits oracle:
activations that are exact multiples of their block's scale give the same
result, any input stays within the quantization bound, and the codes are the
documented rounding (brute force on small blocks)."""
import numpy as np
import pytest

from oracle import int8a as Q8
from oracle import oracle as O


def weights(rng, N, K, bs, zp):
    kb = K // bs
    B = rng.integers(0, 256, (N, kb, bs // 2), dtype=np.uint8)
    S = rng.uniform(0.01, 0.1, (N, kb)).astype(np.float32)
    Z = rng.integers(0, 256, (N, (kb + 1) // 2), dtype=np.uint8) if zp else None
    return B, S, Z


@pytest.mark.parametrize("bs,zp", [(32, False), (64, True), (128, True), (256, False)])
def test_exact_multiples_equal_float32_result(bs, zp):
    rng = np.random.default_rng(bs + zp)
    M, K, N = 3, 512, 24
    B, S, Z = weights(rng, N, K, bs, zp)
    # each block holds integers in [-127, 127] with 127 present, times a power of two
    q = rng.integers(-127, 128, (M, K))
    q[:, ::128] = 127
    A = (q * 2.0 ** rng.integers(-6, 3, (M, K // 128)).repeat(128, axis=1)).astype(np.float32)
    kind = O.ZP_PACKED if zp else None
    got = Q8.matmul_nbits_int8a(A, B, S, Z, K=K, N=N, block_size=bs, zp_kind=kind)
    want = O.matmul_nbits(A, B, S, Z, K=K, N=N, block_size=bs, zp_kind=kind)
    assert np.allclose(got, want, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_within_quantization_bound(dtype):
    rng = np.random.default_rng(7)
    M, K, N, bs = 5, 1024, 40, 64
    B, S, Z = weights(rng, N, K, bs, True)
    A = (rng.standard_normal((M, K)) * rng.uniform(0.1, 10, (M, 1))).astype(dtype)
    got = Q8.matmul_nbits_int8a(A, B, S, Z, K=K, N=N, block_size=bs, zp_kind=O.ZP_PACKED, out_dtype=np.float64)
    want = O.matmul_nbits(A, B, S, Z, K=K, N=N, block_size=bs, zp_kind=O.ZP_PACKED, out_dtype=np.float64)
    bound = Q8.quantization_bound(A, B, S, Z, K=K, block_size=bs, zp_kind=O.ZP_PACKED)
    assert np.all(np.abs(got - want) <= bound * (1 + 1e-9) + 1e-9)
    assert np.abs(got - want).max() > 0  # the path does quantize


def test_codes_brute_force():
    rng = np.random.default_rng(3)
    A = (rng.standard_normal((4, 256)) * 3).astype(np.float32)
    A[1, :128] = 0  # a zero block
    A[2, 5] = -np.abs(A[2, :128]).max() * 2  # the block maximum is negative
    q, s = Q8.quantize_activations(A, 256)
    for m in range(4):
        for b in range(2):
            blk = A[m, 128 * b:128 * (b + 1)]
            sc = np.float32(np.float32(np.abs(blk).max()) / np.float32(127))
            assert s[m, b] == sc
            for i, a in enumerate(blk):
                want = 0 if sc == 0 else int(np.rint(np.float32(a) / sc))
                assert q[m, 128 * b + i] == want
    assert np.all(np.abs(q) <= 127) and q[2, 5] == -127
