"""GPU: float32 MatMulNBits on the float32 GEMV beyond four rows (chunks of
four rows on the grid) and with 8-bit codes (the upstream
qwen3-qproj-decode-m1-q8g32 case's geometry, …/com.microsoft.MatMulNBits/
build/webgpu/bench.json:224), and on the float32 matrix-core GEMM (more than
16 rows, with a workspace), against the oracle at the float32 bar
max|d| <= 1e-5 max|Y_ref|."""
import zlib

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
    (1, 4096, 1000, 2, 32, None, True),         # 2-bit codes: one dword per 16 codes
    (3, 2048, 300, 2, 64, "packed", False),
    (4, 1024, 100, 2, 16, "float", True),
    (16, 4096, 96, 2, 128, "packed", True),
    (2, 8192, 64, 2, 32, None, False),          # two chunks per lane
    (7, 8192, 130, 2, 64, "packed", True),      # two chunks per lane, seven rows: chunks of two rows
    (5, 16384, 40, 2, 32, None, False),         # four chunks per lane: one row per workgroup
]


def want_kernel(M, bs, zp, float16):
    """The family a call with a workspace takes: the float32-arithmetic MFMA
    GEMM beyond 16 rows for blocks of 32 or more, float zero points only of
    the activations' type and with blocks of 64 or more."""
    fz = {"float": not float16, "float16": float16}
    ok = M > 16 and bs >= 32 and (zp not in fz or (fz[zp] and bs >= 64))
    return "gemm_f32_mfma" if ok else "gemv_q4_f32"


def gemv_call(A, B, S, Z, b, M, K, N, bits, bs):
    """The workspace-free entry point: float32 calls take the float32 GEMV at
    every row count."""
    from xrgpu_amd import _native as nat
    tA, tB, tS, tZ, tb = dev(A), dev(B), dev(S), dev(Z), dev(b)
    zdt = nat.UNSPECIFIED if Z is None else {np.uint8: nat.U8, np.float16: nat.F16, np.float32: nat.F32}[Z.dtype.type]
    Y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    nat.check(nat.lib().xrmm_matmul_nbits(ptr(tA), ptr(tB), ptr(tS), ptr(tZ), zdt, ptr(tb), Y.data_ptr(), M, K, N,
                                          bits, bs, nat.F32, None))
    return Y.cpu().numpy()


@pytest.mark.parametrize("M,K,N,bits,bs,zp,bias", CASES)
def test_f32_gemv_parity(gpu, M, K, N, bits, bs, zp, bias):
    rng = np.random.default_rng(M * 11 + K + N + bits + bs)
    A, B, S, Z, b = case(rng, M, K, N, bits, bs, zp, bias)
    kind = None if zp is None else ("packed" if zp == "packed" else "float")
    # more than 16 rows with a workspace (ops supplies one): the matrix-core GEMM
    want = want_kernel(M, bs, zp, False)
    assert ops().select_kernel("MatMulNBits", M, K, N, bits, bs, torch.float32, kind,
                               zp_dtype=torch.float16 if zp == "float16" else None) == want
    Y = ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), dev(b), K=K, N=N, bits=bits, block_size=bs).cpu().numpy()
    ref = O.matmul_nbits(A, B, S, Z, b, K=K, N=N, bits=bits, block_size=bs)
    ok, err, lim = O.tolerance_ok(Y, ref, np.float32)
    assert ok, (err, lim)
    # the workspace-free entry point runs the GEMV at any row count
    ok, err, lim = O.tolerance_ok(gemv_call(A, B, S, Z, b, M, K, N, bits, bs), ref, np.float32)
    assert ok, (err, lim)


MFMA_CASES = [
    # M, K, N, bits, bs, zp, bias: the float32 matrix-core GEMM
    (17, 4096, 4096, 4, 32, None, False),     # 64 tiles: K split in four
    (64, 4096, 4096, 4, 32, "packed", True),
    (100, 2560, 4096, 8, 32, None, True),     # the q8 geometry at prefill rows
    (65, 2048, 300, 8, 64, "packed", False),  # ragged column tile, 64-code blocks
    (130, 1000, 520, 4, 128, "packed", True),  # partial last block (K = 1000)
    (33, 8192, 96, 4, 256, None, False),       # one column tile: four splits of 32 steps
    (48, 6144, 200, 8, 2048, "packed", True),  # blocks of 32 K steps
    (300, 1536, 1024, 4, 64, "packed", False),
    (520, 4096, 2048, 8, 128, None, False),    # many tiles: one split
    (40, 2052, 260, 8, 2048, None, True),      # one 2048-code block, then a partial one
    (64, 2560, 4096, 2, 64, None, False),      # 2-bit codes
    (100, 1000, 300, 2, 32, "packed", True),
    (48, 4096, 520, 2, 256, "packed", False),  # 2-bit blocks of 4 K steps, split K
    (512, 2560, 4096, 4, 64, "float", True),   # upstream qwen3 prefill zero-bias: float zero points
    (64, 1000, 300, 8, 128, "float", False),   # float zero points, partial last block
    (40, 4096, 200, 2, 2048, "float", True),   # float zero points, blocks of 32 K steps, split K
    (48, 2561, 1021, 8, 32, None, False),      # upstream tail case: K % 4 != 0, half a last K step
    (32, 2561, 4096, 4, 32, "packed", True),
    (17, 99, 33, 4, 64, None, True),           # one short K step
    (5, 4096, 8192, 4, 32, "packed", True),    # 2^25 codes: the GEMM from 5 rows
    (12, 4096, 4096, 8, 64, "float", False),   # 2^24 codes: from 12 rows
    (16, 4096, 14336, 2, 64, None, True),
]


@pytest.mark.parametrize("M,K,N,bits,bs,zp,bias", MFMA_CASES)
def test_f32_mfma_gemm_parity(gpu, M, K, N, bits, bs, zp, bias):
    """The float32 matrix-core GEMM against the oracle at the float32 bar, and
    against the float32 GEMV of the workspace-free entry point."""
    rng = np.random.default_rng(M * 7 + K + N + bits + bs)
    A, B, S, Z, b = case(rng, M, K, N, bits, bs, zp, bias)
    assert ops().select_kernel("MatMulNBits", M, K, N, bits, bs, torch.float32, zp) == "gemm_f32_mfma"
    Y = ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), dev(b), K=K, N=N, bits=bits, block_size=bs).cpu().numpy()
    ref = O.matmul_nbits(A, B, S, Z, b, K=K, N=N, bits=bits, block_size=bs)
    ok, err, lim = O.tolerance_ok(Y, ref, np.float32)
    assert ok, (err, lim)
    ok, err, lim = O.tolerance_ok(Y, gemv_call(A, B, S, Z, b, M, K, N, bits, bs), np.float32)
    assert ok, (err, lim)


def test_f32_mfma_row_scaling_extremes(gpu):
    """Rows scaled by powers of ten far from 1 (1e-38 .. 1e36), a row of zeros,
    a row of float32 subnormals, infinities and a NaN. Finite rows: within
    1e-5 of the row's largest exact (float64) output plus half a subnormal
    step (the output's own rounding); non-finite elements as the oracle's
    serial float32 loop gives them (Inf * 0 = NaN on the column whose code
    equals its zero point)."""
    M, K, N, bits, bs = 24, 512, 128, 4, 32
    rng = np.random.default_rng(77)
    A, B, S, Z, b = case(rng, M, K, N, bits, bs, "packed", False)
    scale = np.array([1e-38, 1e-30, 1e-10, 1.0, 1e10, 1e30, 1e36, 2.0 ** -100] * 3, dtype=np.float64)
    A = (A.astype(np.float64) * scale[:, None]).astype(np.float32)
    A[8] = 0.0
    A[9] = np.where(A[9] < 0, -1.0, 1.0).astype(np.float32) * np.float32(1e-44)  # subnormals only
    A[10, 5] = np.inf
    A[11, 100] = -np.inf
    A[12, 7] = np.nan
    B[3, 0, 2] = (B[3, 0, 2] & 0x0F) | 0x80  # k = 5 (high nibble of byte 2): code 8 ...
    Z[3, 0] = (Z[3, 0] & 0xF0) | 8           # ... at zero point 8: W = 0 on column 3
    assert ops().select_kernel("MatMulNBits", M, K, N, bits, bs, torch.float32, "packed") == "gemm_f32_mfma"
    Y = ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), None, K=K, N=N, bits=bits, block_size=bs).cpu().numpy()
    ref = O.matmul_nbits(A, B, S, Z, None, K=K, N=N, bits=bits, block_size=bs)
    bad = (10, 11, 12)
    assert np.array_equal(np.isnan(Y[list(bad)]), np.isnan(ref[list(bad)]))
    inf = np.isinf(ref[list(bad)])
    assert np.array_equal(Y[list(bad)][inf], ref[list(bad)][inf])
    assert np.isnan(Y[10, 3]) and np.isinf(Y[10, 4]) and np.isnan(Y[12]).all()
    fin = [m for m in range(M) if m not in bad]
    exact = O.matmul_nbits(A[fin], B, S, Z, None, K=K, N=N, bits=bits, block_size=bs, out_dtype=np.float64)
    for i, m in enumerate(fin):
        lim = 1e-5 * np.abs(exact[i]).max() + 2.0 ** -150
        assert np.isfinite(Y[m]).all(), m
        assert np.abs(Y[m].astype(np.float64) - exact[i]).max() <= lim, m
    assert np.array_equal(Y[8], np.zeros(N, np.float32))


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
    (2, 5120, 1000, 2, 128, "float16", False),  # 2-bit decode, the bonsai2 K and blocks
    (8, 2048, 200, 2, 32, "packed", True),
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
    want = want_kernel(M, bs, zp, True)
    assert ops().select_kernel("MatMulNBits", M, K, N, bits, bs, torch.float16, kind,
                               zp_dtype=torch.float32 if zp == "float" else None) == want
    Y = ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), dev(b), K=K, N=N, bits=bits, block_size=bs)
    assert Y.dtype == torch.float16
    Y = Y.cpu().numpy()
    ref = O.matmul_nbits(A, B, S, Z, b, K=K, N=N, bits=bits, block_size=bs)
    ok, err, lim = O.tolerance_ok(Y, ref, np.float16)
    assert ok, (err, lim)
    exact = O.matmul_nbits(A, B, S, Z, b, K=K, N=N, bits=bits, block_size=bs, out_dtype=np.float64)
    bound = np.abs(exact) * 2.0 ** -11 + 1e-5 * np.abs(exact).max()
    assert np.all(np.abs(Y.astype(np.float64) - exact) <= bound)


F16_MFMA_CASES = [
    # M, K, N, bits, bs, zp, bias: float16 activations on the float32-arithmetic GEMM
    (512, 2560, 4096, 8, 32, None, False),      # the upstream q8 geometry at 512 rows, float16
    (128, 5120, 1040, 2, 128, "packed", False),  # 2-bit, bonsai2-like (K 5120, blocks of 128)
    (65, 1024, 300, 2, 32, None, True),
    (33, 2048, 96, 8, 64, "packed", True),       # one column tile: K split
    (200, 1000, 257, 8, 256, None, False),       # partial last block (K % 8 == 0)
    (128, 5120, 1040, 2, 128, "float16", False),  # upstream bonsai2: float16 zero points
    (64, 2048, 300, 8, 64, "float16", True),
    (12, 4096, 4096, 8, 32, None, False),        # 2^24 codes: from 12 rows
    (9, 4096, 8192, 2, 64, "float16", True),     # 2^25 codes: from 5 rows
]


@pytest.mark.parametrize("M,K,N,bits,bs,zp,bias", F16_MFMA_CASES)
def test_f16_wide_codes_on_the_mfma_gemm(gpu, M, K, N, bits, bs, zp, bias):
    """float16 activations with 2- or 8-bit codes and more than 16 rows run the
    float32-arithmetic MFMA GEMM: exact binary16 operands (activations, codes
    minus zero points), float32 block sums and scales, one rounding at the
    output, so every element is within one binary16 rounding (2^-11
    relative) plus 1e-5 max|Y| of the exact result."""
    rng = np.random.default_rng(M * 17 + K + N + bits + bs)
    A, B, S, Z, b = case(rng, M, K, N, bits, bs, zp, bias)
    A, S = A.astype(np.float16), S.astype(np.float16)
    b = None if b is None else b.astype(np.float16)
    kind = None if zp is None else ("packed" if zp == "packed" else "float")
    assert ops().select_kernel("MatMulNBits", M, K, N, bits, bs, torch.float16, kind) == "gemm_f32_mfma"
    Y = ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), dev(b), K=K, N=N, bits=bits, block_size=bs)
    assert Y.dtype == torch.float16
    Y = Y.cpu().numpy()
    ref = O.matmul_nbits(A, B, S, Z, b, K=K, N=N, bits=bits, block_size=bs)
    ok, err, lim = O.tolerance_ok(Y, ref, np.float16)
    assert ok, (err, lim)
    exact = O.matmul_nbits(A, B, S, Z, b, K=K, N=N, bits=bits, block_size=bs, out_dtype=np.float64)
    bound = np.abs(exact) * 2.0 ** -11 + 1e-5 * np.abs(exact).max()
    assert np.all(np.abs(Y.astype(np.float64) - exact) <= bound)


@pytest.mark.parametrize("dt,bits,bs,zp", [(np.float32, 4, 64, "float"), (np.float32, 8, 128, "float"),
                                           (np.float16, 2, 128, "float16"), (np.float32, 4, 32, "packed"),
                                           (np.float16, 8, 64, None)])
def test_mfma_gemm_nonfinite_rows(gpu, dt, bits, bs, zp):
    """Rows holding +Inf, -Inf and NaN among finite rows, fractional float zero
    points: with float zero points such rows are recomputed in the
    reference's serial form (the integer / fraction split of z would turn
    Inf * (code - z) into Inf * 0); with integer zero points Inf * (code - z)
    is the reference's product already. Every element matches the oracle:
    non-finite ones exactly, finite rows within the bar."""
    M, K, N = 40, 1024, 300
    rng = np.random.default_rng(bits * 100 + bs)
    A, B, S, Z, _ = case(rng, M, K, N, bits, bs, zp, False)
    A[3, 17] = np.inf
    A[7, 500] = -np.inf
    A[11, 1000] = np.nan
    A[20, 5] = np.inf
    A[20, 6] = -np.inf
    A, S = A.astype(dt), S.astype(dt)
    if zp == "float16":
        Z = Z.astype(np.float16)
    kind = None if zp is None else ("packed" if zp == "packed" else "float")
    assert ops().select_kernel("MatMulNBits", M, K, N, bits, bs, torch.from_numpy(A).dtype, kind) == "gemm_f32_mfma"
    Y = ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), None, K=K, N=N, bits=bits, block_size=bs).cpu().numpy()
    ref = O.matmul_nbits(A, B, S, Z, None, K=K, N=N, bits=bits, block_size=bs)
    ok, err, lim = O.tolerance_ok(Y, ref, dt)
    assert ok, (err, lim, np.argwhere(np.isfinite(Y) != np.isfinite(ref))[:5])
    assert not np.isfinite(ref[3]).any() and np.isnan(ref[11]).all() and np.isfinite(ref[0]).all()


UPSTREAM_PREFILL = [
    # name, M, K, N, bits, bs, zp, activations: the upstream prefill cases at their own sizes
    # (…/com.microsoft.MatMulNBits/build/webgpu/bench.json; inputs drawn here, not the
    # upstream generators)
    ("qwen3-qproj-prefill-m512-q4g64-zero-bias", 512, 2560, 4096, 4, 64, "float", np.float32),
    ("qwen3-qproj-prefill-m512-q8g32", 512, 2560, 4096, 8, 32, None, np.float32),
    ("qwen3-prefill-m512-q8g32-unaligned-n2052", 512, 2560, 2052, 8, 32, None, np.float32),
    ("matmul-nbits-q4-naive-fallback-tailK-m32-k2561-n4096", 32, 2561, 4096, 4, 32, None, np.float32),
    ("rfdetr-fc2-m1300-q4g64", 1300, 1536, 384, 4, 64, None, np.float32),
    ("bonsai2-ffn-gate-prefill-m128-q2g128-k5120-n17408-zero1-f16", 128, 5120, 17408, 2, 128, "float16", np.float16),
]


@pytest.mark.parametrize("name,M,K,N,bits,bs,zp,dt", UPSTREAM_PREFILL, ids=[c[0] for c in UPSTREAM_PREFILL])
def test_upstream_prefill_cases_full_size(gpu, name, M, K, N, bits, bs, zp, dt):
    """The upstream prefill geometries at full size on the float32-arithmetic
    MFMA GEMM, against the oracle at the bar of the activations' type."""
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    A, B, S, Z, b = case(rng, M, K, N, bits, bs, zp, False)
    A = (A * 0.2).astype(dt)
    S = S.astype(dt)
    if zp == "float16":
        Z = Z.astype(np.float16)
    kind = None if zp is None else ("packed" if zp == "packed" else "float")
    assert ops().select_kernel("MatMulNBits", M, K, N, bits, bs, torch.from_numpy(A).dtype, kind) == "gemm_f32_mfma"
    Y = ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), None, K=K, N=N, bits=bits, block_size=bs).cpu().numpy()
    ref = O.matmul_nbits(A, B, S, Z, None, K=K, N=N, bits=bits, block_size=bs)
    ok, err, lim = O.tolerance_ok(Y, ref, dt)
    assert ok, (err, lim)
