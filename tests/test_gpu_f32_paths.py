"""GPU: float32 MatMulNBits on the float32 GEMV beyond four rows (chunks of
four rows on the grid) and with 8-bit codes (the upstream
qwen3-qproj-decode-m1-q8g32 case's geometry, …/com.microsoft.MatMulNBits/
build/webgpu/bench.json:224), against the oracle at the float32 bar
max|d| <= 1e-5 max|Y_ref|."""
import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).cuda()


def ops():
    from xrgpu_amd import ops as _ops
    return _ops


def case(rng, M, K, N, bits, bs, zp, bias):
    kb = O.k_blocks(K, bs)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.integers(0, 256, size=(N, kb, O.blob_bytes(bs, bits)), dtype=np.uint8)
    S = rng.uniform(0.001, 0.02, (N, kb)).astype(np.float32)
    Z = None
    if zp == "packed":
        Z = rng.integers(0, 256, size=(N, O.packed_zp_bytes(kb, bits)), dtype=np.uint8)
    elif zp == "float":
        Z = rng.uniform(0, (1 << bits) - 1, (N, kb)).astype(np.float32)
    elif zp == "float16":
        Z = rng.integers(0, 1 << bits, size=(N, kb)).astype(np.float16)
    b = (rng.standard_normal(N) * 0.1).astype(np.float32) if bias else None
    return A, B, S, Z, b


CASES = [
    # M, K, N, bits, bs, zp, bias
    (1, 2560, 4096, 8, 32, None, False),      # the upstream q8 decode geometry
    (3, 2560, 520, 8, 32, "packed", True),
    (4, 1024, 100, 8, 64, "float", False),
    (2, 512, 64, 8, 16, "float16", True),     # 16-code blocks: one block per chunk
    (5, 2048, 200, 4, 32, "packed", True),    # one row past a chunk
    (17, 1024, 96, 8, 128, None, True),
    (64, 4096, 256, 4, 32, None, False),      # float32 prefill, 16 chunks of four rows
    (130, 768, 72, 8, 32, "packed", False),
]


@pytest.mark.parametrize("M,K,N,bits,bs,zp,bias", CASES)
def test_f32_gemv_parity(gpu, M, K, N, bits, bs, zp, bias):
    rng = np.random.default_rng(M * 11 + K + N + bits + bs)
    A, B, S, Z, b = case(rng, M, K, N, bits, bs, zp, bias)
    kind = None if zp is None else ("packed" if zp == "packed" else "float")
    assert ops().select_kernel("MatMulNBits", M, K, N, bits, bs, torch.float32, kind) == "gemv_q4_f32"
    Y = ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), dev(b), K=K, N=N, bits=bits, block_size=bs).cpu().numpy()
    ref = O.matmul_nbits(A, B, S, Z, b, K=K, N=N, bits=bits, block_size=bs)
    ok, err, lim = O.tolerance_ok(Y, ref, np.float32)
    assert ok, (err, lim)


def test_f32_8bit_infinite_activation(gpu):
    """An infinite activation takes the per-element form on the 8-bit path
    too: +-Inf * W keeps its sign, NaN where W is 0, as the reference's serial
    float32 loop gives."""
    rng = np.random.default_rng(8)
    M, K, N, bits, bs = 2, 256, 64, 8, 32
    A, B, S, Z, b = case(rng, M, K, N, bits, bs, None, False)
    A[1, 37] = np.inf
    B[5, 37 // bs, 37 % bs] = 128  # code == midpoint: W = 0 on column 5
    Y = ops().matmul_nbits(dev(A), dev(B), dev(S), None, None, K=K, N=N, bits=bits, block_size=bs).cpu().numpy()
    ref = O.matmul_nbits(A, B, S, None, None, K=K, N=N, bits=bits, block_size=bs)
    assert O.tolerance_ok(Y, ref, np.float32)[0]
    assert np.isnan(Y[1, 5]) and np.isnan(ref[1, 5])


F16_CASES = [
    # M, K, N, bits, bs, zp, bias: float16 calls with 8-bit codes
    (1, 2560, 4096, 8, 32, None, False),      # the upstream q8 decode geometry in float16
    (3, 2560, 520, 8, 32, "packed", True),
    (4, 1024, 100, 8, 64, "float16", False),
    (17, 1024, 96, 8, 128, None, True),
    (130, 768, 72, 8, 32, "packed", False),
    (512, 256, 64, 8, 16, "float16", True),   # prefill rows, 16-code blocks
]


@pytest.mark.parametrize("M,K,N,bits,bs,zp,bias", F16_CASES)
def test_f16_8bit_on_the_float32_gemv(gpu, M, K, N, bits, bs, zp, bias):
    """float16 MatMulNBits with 8-bit codes runs the float32-arithmetic GEMV:
    activations, scales and bias widen exactly, the sums are float32 and the
    output is rounded once, so every element is within one binary16 rounding
    (2^-11 relative) plus 1e-5 max|Y| of the exact result, well inside the
    float16 bar."""
    rng = np.random.default_rng(M * 13 + K + N + bits + bs)
    A, B, S, Z, b = case(rng, M, K, N, bits, bs, zp, bias)
    A, S = A.astype(np.float16), S.astype(np.float16)
    b = None if b is None else b.astype(np.float16)
    kind = None if zp is None else ("packed" if zp == "packed" else "float")
    assert ops().select_kernel("MatMulNBits", M, K, N, bits, bs, torch.float16, kind) == "gemv_q4_f32"
    Y = ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), dev(b), K=K, N=N, bits=bits, block_size=bs)
    assert Y.dtype == torch.float16
    Y = Y.cpu().numpy()
    ref = O.matmul_nbits(A, B, S, Z, b, K=K, N=N, bits=bits, block_size=bs)
    ok, err, lim = O.tolerance_ok(Y, ref, np.float16)
    assert ok, (err, lim)
    exact = O.matmul_nbits(A, B, S, Z, b, K=K, N=N, bits=bits, block_size=bs, out_dtype=np.float64)
    bound = np.abs(exact) * 2.0 ** -11 + 1e-5 * np.abs(exact).max()
    assert np.all(np.abs(Y.astype(np.float64) - exact) <= bound)
