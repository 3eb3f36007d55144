"""GPU parity: HIP kernels of libxrmm against the oracle on the same seeded inputs.

Bars: dequantized weights and nibble unpacking bit-exact; outputs within
max|d| <= 1e-2*max|Y_ref| for fp16 and 1e-5*max|Y_ref| for fp32
(``oracle.tolerance_ok``); golden fixtures also meet their own atol/rtol.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests import fixture_util as F
from xrgpu_amd import workloads

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).cuda()


def host(t):
    return None if t is None else t.detach().cpu().numpy()


def ops():
    from xrgpu_amd import ops as _ops
    return _ops


def rand_case(rng, M, K, N, bits, bs, dtype, zp, bias=False, scale_lo=0.001, scale_hi=0.02):
    kb = O.k_blocks(K, bs)
    A = rng.standard_normal((M, K)).astype(dtype)
    B = rng.integers(0, 256, size=(N, kb, O.blob_bytes(bs, bits)), dtype=np.uint8)
    S = rng.uniform(scale_lo, scale_hi, (N, kb)).astype(dtype)
    Z = None
    if zp == "packed":
        Z = rng.integers(0, 256, size=(N, O.packed_zp_bytes(kb, bits)), dtype=np.uint8)
    elif zp == "float_int":
        Z = rng.integers(0, 1 << bits, size=(N, kb)).astype(dtype)
    elif zp == "float":
        Z = rng.uniform(0, (1 << bits) - 1, (N, kb)).astype(dtype)
    b = (rng.standard_normal(N) * 0.1).astype(dtype) if bias else None
    return A, B, S, Z, b


def assert_parity(actual, expected, dtype, what=""):
    ok, err, lim = O.tolerance_ok(actual, expected, dtype)
    assert ok, f"{what}: max|d|={err} > {lim}"


# --------------------------------------------------------------------------- dequantisation

@pytest.mark.parametrize("bs", [16, 32, 48, 64, 128])
@pytest.mark.parametrize("zp", [None, "packed", "float_int", "float"])
def test_dequantize_f16_bit_exact(gpu, bs, zp):
    rng = np.random.default_rng(bs * 7 + len(zp or ""))
    K, N = 4 * bs, 37
    _, B, S, Z, _ = rand_case(rng, 1, K, N, 4, bs, np.float16, zp, scale_lo=1e-7, scale_hi=4.0)
    W = host(ops().dequantize(dev(B), dev(S), dev(Z), K=K, block_size=bs, out_dtype=torch.float16))
    ref = O.dequantize(B, S, Z, K, 4, bs, stage="f16")
    assert np.array_equal(W.view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("bits,bs,K", [(4, 32, 128), (2, 16, 80), (8, 32, 70), (4, 8, 24)])
@pytest.mark.parametrize("zp", [None, "packed", "float"])
def test_dequantize_f32_bit_exact(gpu, bits, bs, K, zp):
    rng = np.random.default_rng(bits * 31 + bs + K)
    _, B, S, Z, _ = rand_case(rng, 1, K, 19, bits, bs, np.float32, zp)
    W = host(ops().dequantize(dev(B), dev(S), dev(Z), K=K, bits=bits, block_size=bs, out_dtype=torch.float32))
    ref = O.dequantize(B, S, Z, K, bits, bs, stage="f32")
    assert np.array_equal(W.view(np.uint32), ref.view(np.uint32))


# --------------------------------------------------------------------------- MatMulNBits

FAST_CASES = [
    # M, K, N, bs, zp, bias
    (1, 256, 64, 32, None, False),
    (1, 512, 50, 32, "packed", True),
    (2, 256, 33, 16, "packed", False),
    (4, 1024, 96, 64, "packed", True),
    (7, 384, 48, 128, None, True),
    (16, 512, 80, 32, "float_int", False),
    (16, 288, 17, 32, None, True),       # K tail inside the last block (K % bs != 0)
    (3, 256, 40, 16, "packed", True),    # two blocks per 16-byte chunk
    (9, 512, 70, 32, "packed", True),    # four column tiles per workgroup
]


@pytest.mark.parametrize("M,K,N,bs,zp,bias", FAST_CASES)
def test_gemv_fp16_parity(gpu, M, K, N, bs, zp, bias):
    rng = np.random.default_rng(M * 1000 + K + N + bs)
    A, B, S, Z, b = rand_case(rng, M, K, N, 4, bs, np.float16, zp, bias)
    want = "gemv_q4_dot" if M <= 4 else "gemv_q4_mfma"
    assert ops().select_kernel("MatMulNBits", M, K, N, 4, bs, torch.float16,
                               None if zp is None else ("packed" if zp == "packed" else "float")) == want
    Y = host(ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), dev(b), K=K, N=N, block_size=bs))
    ref = O.matmul_nbits(A, B, S, Z, b, K=K, N=N, block_size=bs)
    assert_parity(Y, ref, np.float16)


DOT_CASES = [
    # M, K, N, bs, zp, bias: every chunk-round count (1, 2, 4, 8), rows 1..4,
    # block sizes 16..128, every zero-point kind, K tails, N below one wave's
    # columns and N not a multiple of a workgroup's
    (1, 1024, 37, 32, None, False),          # 32 chunks: one round, half the lanes idle
    (1, 2048, 64, 64, "packed", True),       # 64 chunks
    (1, 4096, 1000, 32, None, False),        # the decode layout
    (2, 4096, 129, 128, "packed", True),
    (3, 8192, 70, 32, "float_int", True),    # 256 chunks: four rounds, rows padded to 4
    (4, 14336, 33, 64, "packed", False),     # 448 chunks: eight rounds (down projection)
    (4, 16384, 9, 32, None, True),           # 512 chunks, kb = 512
    (1, 288, 17, 32, "packed", True),        # K tail inside the last chunk round
    (2, 320, 5, 64, "float", False),         # K tail inside a block, float zero points
    (1, 256, 1, 16, "packed", True),         # bs = 16: two blocks per chunk, N = 1
    (4, 512, 23, 16, "float", True),
    (1, 4096, 2, 32, None, False),
    (4, 8192, 70, 16, "packed", True),       # four rows on 8 waves x 4 columns, 4 KB scale blocks
    (2, 4096, 100, 32, None, False),         # two rows, the decode layout
]


@pytest.mark.parametrize("M,K,N,bs,zp,bias", DOT_CASES)
def test_gemv_dot_parity(gpu, M, K, N, bs, zp, bias):
    rng = np.random.default_rng(M * 7919 + K + N + bs)
    A, B, S, Z, b = rand_case(rng, M, K, N, 4, bs, np.float16, zp, bias)
    assert ops().select_kernel("MatMulNBits", M, K, N, 4, bs, torch.float16,
                               None if zp is None else ("packed" if zp == "packed" else "float")) == "gemv_q4_dot"
    Y = host(ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), dev(b), K=K, N=N, block_size=bs))
    ref = O.matmul_nbits(A, B, S, Z, b, K=K, N=N, block_size=bs)
    assert_parity(Y, ref, np.float16)


def test_gemv_dot_float32_zero_points(gpu):
    """T3 = float32 zero points with float16 activations (T3 is independent of T1)."""
    rng = np.random.default_rng(77)
    M, K, N, bs = 2, 1024, 40, 32
    A, B, S, _, b = rand_case(rng, M, K, N, 4, bs, np.float16, None, True)
    Z = rng.uniform(0, 15, (N, K // bs)).astype(np.float32)
    Y = host(ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), dev(b), K=K, N=N, block_size=bs))
    assert_parity(Y, O.matmul_nbits(A, B, S, Z, b, K=K, N=N, block_size=bs), np.float16)


F32_CASES = [
    # M, K, N, bs, zp, bias: float32 activations (the contract's T1 = float32)
    # on the float32 GEMV, up to four rows: one to four chunk rounds, block
    # sizes 16 (two blocks per chunk) to 128, every zero-point kind (float
    # zero points as float32 and float16), K tails, N below one wave
    (1, 2048, 2048, 32, "packed", False),   # the CPU-oracle workload's geometry
    (1, 4096, 1000, 32, None, True),
    (2, 4096, 333, 64, "float", False),
    (2, 8192, 70, 128, "packed", True),     # four chunk rounds
    (4, 1024, 96, 16, "float_int", True),
    (4, 288, 17, 32, "packed", False),      # K tail inside the only chunk round
    (1, 100, 5, 32, None, True),            # K tail inside the only block
    (2, 512, 1, 16, "packed", True),        # N = 1
]


# float zero points run as float32 and as float16 (both are the contract's T3)
F32_PARAMS = [c + (np.float32,) for c in F32_CASES] + \
             [c + (np.float16,) for c in F32_CASES if c[4] in ("float", "float_int")]


@pytest.mark.parametrize("M,K,N,bs,zp,bias,zdt", F32_PARAMS)
def test_gemv_fp32_parity(gpu, M, K, N, bs, zp, bias, zdt):
    rng = np.random.default_rng(M * 5 + K + N + bs)
    A, B, S, Z, b = rand_case(rng, M, K, N, 4, bs, np.float32, zp, bias)
    if Z is not None and Z.dtype != np.uint8:
        Z = Z.astype(zdt)
    kind = None if zp is None else ("packed" if zp == "packed" else "float")
    assert ops().select_kernel("MatMulNBits", M, K, N, 4, bs, torch.float32, kind) == "gemv_q4_f32"
    Y = host(ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), dev(b), K=K, N=N, block_size=bs))
    ref = O.matmul_nbits(A, B, S, Z, b, K=K, N=N, block_size=bs)
    assert Y.dtype == np.float32
    assert_parity(Y, ref, np.float32)


GEMM_CASES = [
    # M, K, N, bs, zp, bias: K of neither 64 nor 128 chunks, so the split-K
    # GEMV takes no row chunks: 17 <= M <= 64 runs the thin GEMM (one or two
    # 32-row MFMA tiles), 65 <= M < 128 the 128 x 128 GEMM
    (17, 256, 64, 32, None, False),
    (40, 288, 70, 16, "float", True),       # thin: bs = 16, K tail
    (32, 1056, 200, 32, "packed", True),    # thin: one row tile, a partial last chunk
    (64, 512, 130, 32, "packed", True),
    (96, 288, 40, 32, "packed", True),   # K tail
    (127, 1024, 256, 128, "packed", True),
    (33, 512, 96, 32, "float", True),       # float zero points (the reference's T3)
    (64, 1024, 130, 64, "float_int", False),
    (120, 288, 70, 16, "float", True),      # bs = 16, K tail
]


@pytest.mark.parametrize("M,K,N,bs,zp,bias", GEMM_CASES)
def test_gemm_fp16_parity(gpu, M, K, N, bs, zp, bias):
    rng = np.random.default_rng(M * 7 + K + N + bs)
    A, B, S, Z, b = rand_case(rng, M, K, N, 4, bs, np.float16, zp, bias)
    kind = None if zp is None else ("packed" if zp == "packed" else "float")
    # up to 64 rows the thin GEMM (split-K GEMV geometries aside), above it
    # the 128 x 128 GEMM
    want = "gemm_q4_thin" if M <= 64 else "gemm_q4_mfma"
    assert ops().select_kernel("MatMulNBits", M, K, N, 4, bs, torch.float16, kind) == want
    Y = host(ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), dev(b), K=K, N=N, block_size=bs))
    ref = O.matmul_nbits(A, B, S, Z, b, K=K, N=N, block_size=bs)
    assert_parity(Y, ref, np.float16)


BIG_CASES = [
    # M, K, N, bs, zp, bias for the 256 x 256 GEMM (M >= 128): whole tiles,
    # partial row and column tiles, odd and even K-step counts (the loop runs
    # steps in pairs), K tails inside a block and inside a step, block sizes
    # 16 (two blocks per chunk) to 128, every zero-point kind
    (256, 4096, 512, 128, "packed", True),   # whole tiles, 64 steps
    (128, 288, 40, 32, "packed", True),      # 5 steps (odd), K tail inside the last step
    (300, 576, 300, 32, None, False),        # 9 steps, partial tiles both ways
    (513, 256, 257, 16, "packed", False),    # bs = 16, one row and one column past a tile
    (130, 200, 33, 32, "packed", True),      # K = 200 inside a block: kb = 7, 4 steps
    (160, 1024, 96, 64, "float_int", True),  # float zero points with integer values
    (140, 512, 72, 128, "float", False),     # float zero points of any value
    (129, 320, 100, 64, None, False),
    (200, 1024, 256, 128, "packed", True),
    # more tiles than CUs: 256-wide then 192-wide tiles on one grid
    (256, 64, 65836, 64, "packed", True),    # 258 tile columns; narrow tiles partial and past N
    (512, 128, 33768, 128, None, True),      # two row tiles of wide + narrow tiles
]


ODD_ZP_CASES = [
    # M, K, N, bs: packed zero-point rows of an odd byte count (ceil(kb / 2)
    # odd), so a column's zero points start at any byte offset
    (1, 864, 64, 64),      # kb 14: 7-byte rows
    (2, 11008, 40, 128),   # kb 86: 43-byte rows (a 7B-class down projection)
    (1, 640, 100, 64),     # kb 10: 5-byte rows
    (4, 11008, 36, 128),
    (8, 11008, 48, 128),
    (64, 864, 200, 64),
    (300, 11008, 72, 128),
    (16, 1056, 200, 16),   # the MFMA GEMV: 33-byte rows, tile staging from odd offsets
    (9, 2080, 77, 32),
    (12, 1312, 100, 32),   # 21-byte rows
]


@pytest.mark.parametrize("M,K,N,bs", ODD_ZP_CASES)
def test_packed_zero_points_odd_rows(gpu, M, K, N, bs):
    rng = np.random.default_rng(M * 17 + K + N + bs)
    A, B, S, Z, b = rand_case(rng, M, K, N, 4, bs, np.float16, "packed", True)
    assert Z.shape[1] % 2 == 1
    Y = host(ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), dev(b), K=K, N=N, block_size=bs))
    kern = ops().select_kernel("MatMulNBits", M, K, N, 4, bs, torch.float16, "packed")
    assert_parity(Y, O.matmul_nbits(A, B, S, Z, b, K=K, N=N, block_size=bs), np.float16, kern)


@pytest.fixture
def big_gemm(monkeypatch):
    """Shapes below the 256 x 256 GEMM's tile threshold reach it through
    XRMM_GEMM_BIG_MIN_TILES = 0, so its edge cases stay small."""
    monkeypatch.setenv("XRMM_GEMM_BIG_MIN_TILES", "0")


@pytest.mark.parametrize("M,K,N,bs,zp,bias", BIG_CASES)
def test_gemm_big_parity(gpu, big_gemm, M, K, N, bs, zp, bias):
    rng = np.random.default_rng(M * 31 + K + N + bs)
    A, B, S, Z, b = rand_case(rng, M, K, N, 4, bs, np.float16, zp, bias)
    kind = None if zp is None else ("packed" if zp == "packed" else "float")
    assert ops().select_kernel("MatMulNBits", M, K, N, 4, bs, torch.float16, kind) == "gemm_q4_big"
    Y = host(ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), dev(b), K=K, N=N, block_size=bs))
    ref = O.matmul_nbits(A, B, S, Z, b, K=K, N=N, block_size=bs)
    assert_parity(Y, ref, np.float16)


def test_gemm_big_float32_zero_points(gpu, big_gemm):
    """T3 = float32 zero points with float16 activations on the 256 x 256 GEMM."""
    rng = np.random.default_rng(78)
    M, K, N, bs = 192, 1024, 80, 32
    A, B, S, _, b = rand_case(rng, M, K, N, 4, bs, np.float16, None, True)
    Z = rng.uniform(0, 15, (N, K // bs)).astype(np.float32)
    Y = host(ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), dev(b), K=K, N=N, block_size=bs))
    assert_parity(Y, O.matmul_nbits(A, B, S, Z, b, K=K, N=N, block_size=bs), np.float16)


def test_gemm_big_repeat_and_rows_independent(gpu, big_gemm):
    """Two launches give identical bytes, and row r of a 384-row product equals
    the same row computed within a 128-row product (rows never mix)."""
    rng = np.random.default_rng(79)
    M, K, N, bs = 384, 512, 200, 32
    A, B, S, Z, b = rand_case(rng, M, K, N, 4, bs, np.float16, "packed", True)
    args = (dev(B), dev(S), dev(Z), dev(b))
    y1 = host(ops().matmul_nbits(dev(A), *args, K=K, N=N, block_size=bs))
    y2 = host(ops().matmul_nbits(dev(A), *args, K=K, N=N, block_size=bs))
    assert np.array_equal(y1.view(np.uint16), y2.view(np.uint16))
    y3 = host(ops().matmul_nbits(dev(A[256:]), *args, K=K, N=N, block_size=bs))
    assert np.array_equal(y1[256:].view(np.uint16), y3.view(np.uint16))


GENERIC_CASES = [
    # M, K, N, bits, bs, dtype, zp, bias
    (1, 2048, 64, 4, 32, np.float32, "packed", False),
    (3, 70, 9, 4, 32, np.float32, "float", True),
    (2, 33, 5, 2, 16, np.float32, None, True),
    (5, 40, 7, 8, 16, np.float16, "packed", False),
    (4, 24, 6, 4, 8, np.float16, None, True),
    (20, 100, 11, 8, 32, np.float32, "float", True),
    (2, 17, 2, 4, 16, np.float16, "float", True),
    (3, 256, 40, 4, 48, np.float16, "packed", False),  # non-power-of-two block
]


@pytest.mark.parametrize("M,K,N,bits,bs,dtype,zp,bias", GENERIC_CASES)
def test_generic_parity(gpu, M, K, N, bits, bs, dtype, zp, bias):
    rng = np.random.default_rng(M + K + N + bits + bs)
    A, B, S, Z, b = rand_case(rng, M, K, N, bits, bs, dtype, zp, bias)
    Y = host(ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), dev(b), K=K, N=N, bits=bits, block_size=bs))
    ref = O.matmul_nbits(A, B, S, Z, b, K=K, N=N, bits=bits, block_size=bs)
    assert_parity(Y, ref, dtype)


def test_rank3_activation_folds_leading_axes(gpu):
    rng = np.random.default_rng(5)
    A, B, S, Z, b = rand_case(rng, 6, 256, 32, 4, 32, np.float16, "packed", True)
    A3 = A.reshape(2, 3, 256)
    Y = host(ops().matmul_nbits(dev(A3), dev(B), dev(S), dev(Z), dev(b), block_size=32))
    assert Y.shape == (2, 3, 32)
    assert_parity(Y, O.matmul_nbits(A3, B, S, Z, b, K=256, N=32, block_size=32), np.float16)


# --------------------------------------------------------------------------- golden fixtures

MNB = "com.microsoft.MatMulNBits"


def run_mnb_fixture(case, ins):
    at = case["attrs"]
    return host(ops().matmul_nbits(dev(ins["aT"]), dev(ins["bT"]), dev(ins["scalesT"]), dev(ins.get("zeroPointsT")),
                                   dev(ins.get("biasT")), K=at["K"], N=at["N"], bits=at.get("bits", 4),
                                   block_size=at["block_size"]))


@pytest.mark.parametrize("name", ["q4_block512_schema_legal_cpu_provider_gap_exact", "empty_zero_dim",
                                  "empty_zero_dim_f16"])
def test_fixture_explicit_outputs(gpu, name):
    case = F.find(MNB, name)
    y = run_mnb_fixture(case, F.case_inputs(case))
    exp = F.materialize(case["outputs"]["yT"])
    assert y.shape == exp.shape and y.dtype == exp.dtype
    assert F.reference_compare(y, exp, *F.case_tolerance(case, "yT"))


@pytest.mark.parametrize("name", ["ort_f16_large_k_accumulator_cancellation_m1_k8192_n8",
                                  "ort_f16_large_k_accumulator_cancellation_m8_k8192_n8",
                                  "f16_full_k_accumulator_cancellation_prefill_m64_k4096_n64"])
def test_fixture_accumulator_cancellation_exact_zero(gpu, name):
    case = F.find(MNB, name)
    y = run_mnb_fixture(case, F.case_inputs(case))
    assert y.dtype == np.float16 and np.all(y == 0), np.abs(y).max()


def test_fixture_shapes_with_oracle(gpu):
    """Every MatMulNBits fixture case of the reference, with its own shapes,
    attributes and data where materialisable (seeded substitutes for the
    upstream-only fillFloat32 generator), against the oracle."""
    ran = 0
    for case in F.load_cases():
        if case["operation"] != MNB:
            continue
        at = case["attrs"]
        ins = F.case_inputs(case, substitute=True)
        if any(v.size > 8_000_000 for v in ins.values()):
            continue
        y = run_mnb_fixture(case, ins)
        ref = O.matmul_nbits(ins["aT"], ins["bT"], ins["scalesT"], ins.get("zeroPointsT"), ins.get("biasT"),
                             K=at["K"], N=at["N"], bits=at.get("bits", 4), block_size=at["block_size"])
        assert_parity(y, ref, ref.dtype, case["name"])
        ran += 1
    assert ran >= 60


SPLITK_CASES = [
    # M, K, N, bs, zp, bias on the split-K GEMV (4 < M <= 16, a column's chunks
    # split evenly over 8 waves x 4 lane groups): chunks per lane 2 and 4,
    # 1, 2 or 4 blocks per lane (and blocks shared by lanes), every zero-point
    # kind, N below one tile, tile counts that leave the last workgroup short
    (8, 4096, 1000, 32, None, False),        # four blocks per lane
    (16, 4096, 333, 64, "packed", True),     # two blocks per lane
    (5, 2048, 70, 32, "float", True),        # two chunks per lane
    (12, 4096, 16, 128, "packed", False),    # one block per lane, odd first blocks
    (16, 2048, 4100, 256, "float_int", True),  # blocks shared by lane groups; 257 tiles
    (7, 4096, 8200, 32, None, True),         # 513 tiles: three per workgroup, last one short
    (16, 4096, 3, 32, "packed", True),       # N below one tile
]


@pytest.mark.parametrize("M,K,N,bs,zp,bias", SPLITK_CASES)
def test_gemv_splitk_parity(gpu, M, K, N, bs, zp, bias):
    rng = np.random.default_rng(M * 977 + K + N + bs)
    A, B, S, Z, b = rand_case(rng, M, K, N, 4, bs, np.float16, zp, bias)
    assert ops().select_kernel("MatMulNBits", M, K, N, 4, bs, torch.float16,
                               None if zp is None else ("packed" if zp == "packed" else "float")) == "gemv_q4_splitk"
    Y = host(ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), dev(b), K=K, N=N, block_size=bs))
    ref = O.matmul_nbits(A, B, S, Z, b, K=K, N=N, block_size=bs)
    assert_parity(Y, ref, np.float16)


def test_gemv_splitk_float32_zero_points(gpu):
    rng = np.random.default_rng(4242)
    M, K, N, bs = 9, 4096, 130, 64
    A, B, S, _, b = rand_case(rng, M, K, N, 4, bs, np.float16, None, True)
    Z = rng.uniform(0, 15, (N, K // bs)).astype(np.float32)
    Y = host(ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), dev(b), K=K, N=N, block_size=bs))
    ref = O.matmul_nbits(A, B, S, Z, b, K=K, N=N, block_size=bs)
    assert_parity(Y, ref, np.float16)


# --------------------------------------------------------------------------- Qkv / Mlp

QKV_CASES = [
    # M, K, Nq, Nkv, bs, dtype, zp, skip
    (1, 256, 64, 32, 32, np.float16, None, False),
    (4, 512, 128, 48, 64, np.float16, "packed", True),
    (16, 256, 40, 24, 32, np.float16, None, True),
    (3, 96, 20, 12, 32, np.float32, "packed", True),
]


@pytest.mark.parametrize("M,K,Nq,Nkv,bs,dtype,zp,skip", QKV_CASES)
def test_qkv_parity(gpu, M, K, Nq, Nkv, bs, dtype, zp, skip):
    rng = np.random.default_rng(M + K + Nq + Nkv)
    A = rng.standard_normal((M, K)).astype(dtype)
    sk = rng.standard_normal((M, K)).astype(dtype) if skip else None
    g = rng.uniform(0.5, 1.5, K).astype(dtype)
    parts = [rand_case(rng, 1, K, n, 4, bs, dtype, zp)[1:4] for n in (Nq, Nkv, Nkv)]
    o = ops()
    Q, Kk, V, R = o.matmul_nbits_qkv(dev(A), *[dev(x) for p in parts for x in p[:2]], norm_scale=dev(g), skip=dev(sk),
                                     block_size=bs, q_zero_points=dev(parts[0][2]), k_zero_points=dev(parts[1][2]),
                                     v_zero_points=dev(parts[2][2]))
    ref = O.matmul_nbits_qkv(A, parts[0][0], parts[0][1], parts[1][0], parts[1][1], parts[2][0], parts[2][1], K=K,
                             Nq=Nq, Nkv=Nkv, norm_scale=g, skip=sk, block_size=bs, q_zero_points=parts[0][2],
                             k_zero_points=parts[1][2], v_zero_points=parts[2][2])
    for got, exp, nm in zip((Q, Kk, V), ref[:3], "qkv"):
        assert_parity(host(got), exp, dtype, nm)
    assert np.array_equal(host(R), ref[3])  # residual A + skip: bit-exact


QKV_DOT_CASES = [
    # M, K, Nq, Nkv, bs, zp, skip for up to four rows: the four-row MFMA GEMV
    # (integer zero points, block_size >= 32, K <= 4096) or else the dot GEMV;
    # every chunk-round count, rows 1..4, bs 16..256, every zero-point kind, K
    # tails, column counts that leave a projection's last tile or wave partly
    # empty
    (4, 4096, 256, 64, 64, "packed", False),   # the GQA decode layout, narrower
    (2, 2048, 96, 40, 32, None, True),
    (3, 8192, 33, 17, 32, "float", True),      # four chunk rounds, odd widths (dot)
    (1, 1024, 20, 12, 16, "packed", True),     # bs = 16: two blocks per chunk (dot)
    (4, 288, 40, 24, 32, "float_int", True),   # K tail inside the only chunk round (dot)
    (4, 16384, 64, 32, 64, None, False),       # eight chunk rounds (dot)
    (1, 64, 1, 1, 32, None, True),             # one column per projection
    (4, 1024, 33, 17, 128, "packed", True),    # odd widths, four chunks per block
    (4, 4096, 16, 16, 256, "packed", False),   # eight chunks per block
    (2, 96, 20, 12, 32, "packed", True),       # three blocks: odd packed zero-point rows
    (3, 4000, 48, 16, 32, None, True),         # K tail inside the last block
]


def qkv_gemv_family(M, K, bs, zp):
    return "gemv_q4_mq" if bs >= 32 and zp in (None, "packed") and K <= 4096 else "gemv_q4_dot"


@pytest.mark.parametrize("M,K,Nq,Nkv,bs,zp,skip", QKV_DOT_CASES)
def test_qkv_dot_parity(gpu, M, K, Nq, Nkv, bs, zp, skip):
    rng = np.random.default_rng(M * 131 + K + Nq + Nkv + bs)
    dt = np.float16
    A = rng.standard_normal((M, K)).astype(dt)
    sk = rng.standard_normal((M, K)).astype(dt) if skip else None
    g = rng.uniform(0.5, 1.5, K).astype(dt)
    parts = [rand_case(rng, 1, K, n, 4, bs, dt, zp)[1:4] for n in (Nq, Nkv, Nkv)]
    kind = None if zp is None else ("packed" if zp == "packed" else "float")
    o = ops()
    assert o.select_kernel("MatMulNBitsQkv", M, K, Nq, 4, bs, torch.float16, kind) == qkv_gemv_family(M, K, bs, zp)
    Q, Kk, V, R = o.matmul_nbits_qkv(dev(A), *[dev(x) for p in parts for x in p[:2]], norm_scale=dev(g), skip=dev(sk),
                                     block_size=bs, q_zero_points=dev(parts[0][2]), k_zero_points=dev(parts[1][2]),
                                     v_zero_points=dev(parts[2][2]))
    ref = O.matmul_nbits_qkv(A, parts[0][0], parts[0][1], parts[1][0], parts[1][1], parts[2][0], parts[2][1], K=K,
                             Nq=Nq, Nkv=Nkv, norm_scale=g, skip=sk, block_size=bs, q_zero_points=parts[0][2],
                             k_zero_points=parts[1][2], v_zero_points=parts[2][2])
    for got, exp, nm in zip((Q, Kk, V), ref[:3], "qkv"):
        assert_parity(host(got), exp, dt, nm)
    assert np.array_equal(host(R), ref[3])  # residual A + skip: bit-exact


QKV_SPLITK_CASES = [
    # M, K, Nq, Nkv, bs, zp, skip on the split-K GEMV (5 <= M <= 16)
    (8, 4096, 256, 64, 64, "packed", True),
    (16, 2048, 40, 24, 32, None, False),
    (6, 4096, 100, 36, 128, "float", True),
]


@pytest.mark.parametrize("M,K,Nq,Nkv,bs,zp,skip", QKV_SPLITK_CASES)
def test_qkv_splitk_parity(gpu, M, K, Nq, Nkv, bs, zp, skip):
    rng = np.random.default_rng(M * 313 + K + Nq + Nkv + bs)
    dt = np.float16
    A = rng.standard_normal((M, K)).astype(dt)
    sk = rng.standard_normal((M, K)).astype(dt) if skip else None
    g = rng.uniform(0.5, 1.5, K).astype(dt)
    parts = [rand_case(rng, 1, K, n, 4, bs, dt, zp)[1:4] for n in (Nq, Nkv, Nkv)]
    kind = None if zp is None else ("packed" if zp == "packed" else "float")
    o = ops()
    assert o.select_kernel("MatMulNBitsQkv", M, K, Nq, 4, bs, torch.float16, kind) == "gemv_q4_splitk"
    Q, Kk, V, R = o.matmul_nbits_qkv(dev(A), *[dev(x) for p in parts for x in p[:2]], norm_scale=dev(g), skip=dev(sk),
                                     block_size=bs, q_zero_points=dev(parts[0][2]), k_zero_points=dev(parts[1][2]),
                                     v_zero_points=dev(parts[2][2]))
    ref = O.matmul_nbits_qkv(A, parts[0][0], parts[0][1], parts[1][0], parts[1][1], parts[2][0], parts[2][1], K=K,
                             Nq=Nq, Nkv=Nkv, norm_scale=g, skip=sk, block_size=bs, q_zero_points=parts[0][2],
                             k_zero_points=parts[1][2], v_zero_points=parts[2][2])
    for got, exp, nm in zip((Q, Kk, V), ref[:3], "qkv"):
        assert_parity(host(got), exp, dt, nm)
    assert np.array_equal(host(R), ref[3])  # residual A + skip: bit-exact


MLP_SPLITK_CASES = [
    # M, K, N, bs, skip, norm, biases, act, residual on the split-K GEMV
    (16, 4096, 1000, 32, False, False, False, "silu", False),   # the batched SwiGLU layout, narrower
    (8, 2048, 72, 64, True, True, True, "silu", True),
    (12, 4096, 40, 32, True, False, False, "gelu", True),
    (5, 4096, 33, 128, False, True, False, "relu", False),
    (16, 4096, 7, 32, False, False, True, "silu", True),       # N below one tile; residual = A
]


@pytest.mark.parametrize("M,K,N,bs,skip,norm,biases,act,res", MLP_SPLITK_CASES)
def test_mlp_splitk_parity(gpu, M, K, N, bs, skip, norm, biases, act, res):
    rng = np.random.default_rng(M * 29 + K + N + bs)
    dt = np.float16
    A = rng.standard_normal((M, K)).astype(dt)
    sk = rng.standard_normal((M, K)).astype(dt) if skip else None
    g = rng.uniform(0.5, 1.5, K).astype(dt) if norm else None
    _, gB, gS, _, gb = rand_case(rng, 1, K, N, 4, bs, dt, None, biases)
    _, uB, uS, _, ub = rand_case(rng, 1, K, N, 4, bs, dt, None, biases)
    assert ops().select_kernel("MatMulNBitsMlp", M, K, N, 4, bs, torch.float16) == "gemv_q4_splitk"
    Y, R = ops().matmul_nbits_mlp(dev(A), dev(gB), dev(gS), dev(uB), dev(uS), skip=dev(sk), norm_scale=dev(g),
                                  gate_bias=dev(gb), up_bias=dev(ub), block_size=bs, activation=act,
                                  want_residual=res)
    ref, r = O.matmul_nbits_mlp(A, gB, gS, uB, uS, K=K, N=N, skip=sk, norm_scale=g, gate_bias=gb, up_bias=ub,
                                block_size=bs, activation=act)
    assert_parity(host(Y), ref, dt)
    if res:
        assert np.array_equal(host(R), r)


MLP_CASES = [
    # M, K, N, bs, dtype, skip, norm, biases, act
    (1, 256, 64, 32, np.float16, False, False, False, "silu"),
    (16, 512, 72, 32, np.float16, False, False, False, "silu"),
    (4, 256, 40, 64, np.float16, True, True, True, "silu"),
    (8, 128, 24, 32, np.float16, True, False, True, "gelu"),
    (2, 64, 10, 16, np.float32, True, True, True, "silu"),
    (5, 256, 33, 32, np.float16, False, True, False, "relu"),
]


@pytest.mark.parametrize("M,K,N,bs,dtype,skip,norm,biases,act", MLP_CASES)
def test_mlp_parity(gpu, M, K, N, bs, dtype, skip, norm, biases, act):
    rng = np.random.default_rng(M + K + N + bs)
    A = rng.standard_normal((M, K)).astype(dtype)
    sk = rng.standard_normal((M, K)).astype(dtype) if skip else None
    g = rng.uniform(0.5, 1.5, K).astype(dtype) if norm else None
    _, gB, gS, _, gb = rand_case(rng, 1, K, N, 4, bs, dtype, None, biases)
    _, uB, uS, _, ub = rand_case(rng, 1, K, N, 4, bs, dtype, None, biases)
    Y, R = ops().matmul_nbits_mlp(dev(A), dev(gB), dev(gS), dev(uB), dev(uS), skip=dev(sk), norm_scale=dev(g),
                                  gate_bias=dev(gb), up_bias=dev(ub), block_size=bs, activation=act,
                                  want_residual=True)
    ref, r = O.matmul_nbits_mlp(A, gB, gS, uB, uS, K=K, N=N, skip=sk, norm_scale=g, gate_bias=gb, up_bias=ub,
                                block_size=bs, activation=act)
    assert_parity(host(Y), ref, dtype)
    assert np.array_equal(host(R), r)


QKV_GEMM_CASES = [
    # M, K, Nq, Nkv, bs, zp, skip on the fused 128 x 128 GEMM (M > 16): row
    # tiles full and partial, projections narrower than one column tile, K
    # tails inside a K step, every zero-point kind, bs 16..128
    (80, 2048, 512, 128, 32, "packed", True),   # GQA prefill layout, narrower
    (17, 1024, 40, 24, 64, None, False),       # one row past the GEMVs, odd widths
    (200, 4096, 256, 64, 128, "float", True),  # two row tiles, the second partial
    (130, 512, 130, 3, 16, "packed", True),    # bs = 16; a 3-column projection
    (33, 96, 20, 12, 32, "float_int", True),   # K = 96: half a K step at the end
    (48, 1000, 136, 8, 64, None, True),        # K = 1000 padded to 1024 by the blocks
]


@pytest.mark.parametrize("M,K,Nq,Nkv,bs,zp,skip", QKV_GEMM_CASES)
def test_qkv_gemm_parity(gpu, M, K, Nq, Nkv, bs, zp, skip):
    rng = np.random.default_rng(M * 7 + K + Nq + Nkv + bs)
    dt = np.float16
    A = rng.standard_normal((M, K)).astype(dt)
    sk = rng.standard_normal((M, K)).astype(dt) if skip else None
    g = rng.uniform(0.5, 1.5, K).astype(dt)
    parts = [rand_case(rng, 1, K, n, 4, bs, dt, zp)[1:4] for n in (Nq, Nkv, Nkv)]
    kind = None if zp is None else ("packed" if zp == "packed" else "float")
    o = ops()
    assert o.select_kernel("MatMulNBitsQkv", M, K, Nq, 4, bs, torch.float16, kind) == "gemm_q4_fused"
    Q, Kk, V, R = o.matmul_nbits_qkv(dev(A), *[dev(x) for p in parts for x in p[:2]], norm_scale=dev(g), skip=dev(sk),
                                     block_size=bs, q_zero_points=dev(parts[0][2]), k_zero_points=dev(parts[1][2]),
                                     v_zero_points=dev(parts[2][2]))
    ref = O.matmul_nbits_qkv(A, parts[0][0], parts[0][1], parts[1][0], parts[1][1], parts[2][0], parts[2][1], K=K,
                             Nq=Nq, Nkv=Nkv, norm_scale=g, skip=sk, block_size=bs, q_zero_points=parts[0][2],
                             k_zero_points=parts[1][2], v_zero_points=parts[2][2])
    for got, exp, nm in zip((Q, Kk, V), ref[:3], "qkv"):
        assert_parity(host(got), exp, dt, nm)
    assert np.array_equal(host(R), ref[3])  # residual A + skip: bit-exact


MLP_GEMM_CASES = [
    # M, K, N, bs, zp, skip, norm, biases, act, residual on the fused GEMM
    (72, 2048, 5632, 32, None, False, True, False, "silu", True),   # the SwiGLU prefill layout
    (17, 1024, 72, 64, "packed", True, True, True, "silu", True),
    (130, 512, 33, 32, None, True, False, True, "gelu", True),       # N below one 64-output tile
    (70, 4096, 100, 128, "float", False, False, False, "relu", False),
    (256, 992, 64, 16, "packed", True, True, True, "tanh", True),    # bs = 16; K ends half way into a step
    (24, 256, 96, 32, None, False, True, True, "sigmoid", False),
    (24, 256, 96, 32, "float_int", True, False, True, "none", True),
    (24, 256, 96, 32, None, True, True, False, "swiglu", False),
    (64, 2048, 5632, 32, None, False, True, False, "silu", False),  # the 64-row SwiGLU prefill leg
    (40, 512, 130, 16, "packed", True, True, True, "silu", True),   # bs = 16, a partial last tile
]


@pytest.mark.parametrize("M,K,N,bs,zp,skip,norm,biases,act,res", MLP_GEMM_CASES)
def test_mlp_gemm_parity(gpu, M, K, N, bs, zp, skip, norm, biases, act, res):
    rng = np.random.default_rng(M * 37 + K + N + bs)
    dt = np.float16
    A = rng.standard_normal((M, K)).astype(dt)
    sk = rng.standard_normal((M, K)).astype(dt) if skip else None
    g = rng.uniform(0.5, 1.5, K).astype(dt) if norm else None
    _, gB, gS, gZ, gb = rand_case(rng, 1, K, N, 4, bs, dt, zp, biases)
    _, uB, uS, uZ, ub = rand_case(rng, 1, K, N, 4, bs, dt, zp, biases)
    kind = None if zp is None else ("packed" if zp == "packed" else "float")
    want = "gemm_q4_thin" if M <= 64 else "gemm_q4_fused"  # 17..64 rows: the thin GEMM
    assert ops().select_kernel("MatMulNBitsMlp", M, K, N, 4, bs, torch.float16, kind) == want
    Y, R = ops().matmul_nbits_mlp(dev(A), dev(gB), dev(gS), dev(uB), dev(uS), skip=dev(sk), norm_scale=dev(g),
                                  gate_bias=dev(gb), up_bias=dev(ub), block_size=bs, activation=act,
                                  gate_zero_points=dev(gZ), up_zero_points=dev(uZ), want_residual=res)
    ref, r = O.matmul_nbits_mlp(A, gB, gS, uB, uS, K=K, N=N, skip=sk, norm_scale=g, gate_bias=gb, up_bias=ub,
                                block_size=bs, activation=act, gate_zero_points=gZ, up_zero_points=uZ)
    assert_parity(host(Y), ref, dt)
    if res:
        assert np.array_equal(host(R), r)


SK_CHUNK_CASES = [
    # op, M, K, N (Qkv: Nq, Nkv), bs, zp, extras: the split-K GEMV over row
    # chunks of 16 (17..64 rows, K of 64 or 128 chunks): partial last chunks,
    # every operator and zero-point kind, prologue and epilogue variants (Mlp
    # runs the thin GEMM at these rows, after the same prologue)
    ("mnb", 17, 4096, 100, 32, "packed", dict(bias=True)),
    ("mnb", 33, 2048, 260, 64, "float", dict(bias=True)),
    ("mnb", 64, 4096, 1000, 128, None, dict(bias=False)),
    ("mnb", 48, 2048, 33, 32, "float_int", dict(bias=True)),
    ("qkv", 40, 4096, (256, 64), 64, "packed", dict(skip=True)),
    ("qkv", 64, 2048, (100, 36), 32, None, dict(skip=False)),
    ("mlp", 24, 2048, 96, 32, None, dict(skip=True, norm=True, biases=True, act="silu", res=True)),
    ("mlp", 64, 4096, 40, 64, "packed", dict(skip=False, norm=True, biases=False, act="gelu", res=False)),
    ("mlp", 50, 2048, 33, 128, None, dict(skip=True, norm=False, biases=True, act="relu", res=True)),
]


@pytest.mark.parametrize("op,M,K,N,bs,zp,ex", SK_CHUNK_CASES)
def test_splitk_row_chunks(gpu, op, M, K, N, bs, zp, ex):
    rng = np.random.default_rng(M * 53 + K + bs + len(op))
    dt = np.float16
    o = ops()
    kind = None if zp is None else ("packed" if zp == "packed" else "float")
    A = rng.standard_normal((M, K)).astype(dt)
    if op == "mnb":
        _, B, S, Z, b = rand_case(rng, M, K, N, 4, bs, dt, zp, ex["bias"])
        assert o.select_kernel("MatMulNBits", M, K, N, 4, bs, torch.float16, kind) == "gemv_q4_splitk"
        Y = host(o.matmul_nbits(dev(A), dev(B), dev(S), dev(Z), dev(b), K=K, N=N, block_size=bs))
        assert_parity(Y, O.matmul_nbits(A, B, S, Z, b, K=K, N=N, block_size=bs), dt)
    elif op == "qkv":
        Nq, Nkv = N
        sk = rng.standard_normal((M, K)).astype(dt) if ex["skip"] else None
        g = rng.uniform(0.5, 1.5, K).astype(dt)
        parts = [rand_case(rng, 1, K, n, 4, bs, dt, zp)[1:4] for n in (Nq, Nkv, Nkv)]
        assert o.select_kernel("MatMulNBitsQkv", M, K, Nq, 4, bs, torch.float16, kind) == "gemv_q4_splitk"
        Q, Kk, V, R = o.matmul_nbits_qkv(dev(A), *[dev(x) for p in parts for x in p[:2]], norm_scale=dev(g),
                                         skip=dev(sk), block_size=bs, q_zero_points=dev(parts[0][2]),
                                         k_zero_points=dev(parts[1][2]), v_zero_points=dev(parts[2][2]))
        ref = O.matmul_nbits_qkv(A, parts[0][0], parts[0][1], parts[1][0], parts[1][1], parts[2][0], parts[2][1],
                                 K=K, Nq=Nq, Nkv=Nkv, norm_scale=g, skip=sk, block_size=bs,
                                 q_zero_points=parts[0][2], k_zero_points=parts[1][2], v_zero_points=parts[2][2])
        for got, exp, nm in zip((Q, Kk, V), ref[:3], "qkv"):
            assert_parity(host(got), exp, dt, nm)
        assert np.array_equal(host(R), ref[3])  # residual A + skip: bit-exact, every row chunk
    else:
        sk = rng.standard_normal((M, K)).astype(dt) if ex["skip"] else None
        g = rng.uniform(0.5, 1.5, K).astype(dt) if ex["norm"] else None
        _, gB, gS, gZ, gb = rand_case(rng, 1, K, N, 4, bs, dt, zp, ex["biases"])
        _, uB, uS, uZ, ub = rand_case(rng, 1, K, N, 4, bs, dt, zp, ex["biases"])
        assert o.select_kernel("MatMulNBitsMlp", M, K, N, 4, bs, torch.float16, kind) == "gemm_q4_thin"
        Y, R = o.matmul_nbits_mlp(dev(A), dev(gB), dev(gS), dev(uB), dev(uS), skip=dev(sk), norm_scale=dev(g),
                                  gate_bias=dev(gb), up_bias=dev(ub), block_size=bs, activation=ex["act"],
                                  gate_zero_points=dev(gZ), up_zero_points=dev(uZ), want_residual=ex["res"])
        ref, r = O.matmul_nbits_mlp(A, gB, gS, uB, uS, K=K, N=N, skip=sk, norm_scale=g, gate_bias=gb, up_bias=ub,
                                    block_size=bs, activation=ex["act"], gate_zero_points=gZ, up_zero_points=uZ)
        assert_parity(host(Y), ref, dt)
        if ex["res"]:
            assert np.array_equal(host(R), r)


def test_gemm_fused_rows_independent(gpu):
    """A row's outputs do not depend on the other rows of its tile (each row's
    normalisation factor is its own) and a repeat gives the same bits."""
    rng = np.random.default_rng(5)
    M, K, N, bs = 96, 1024, 160, 32
    A = rng.standard_normal((M, K)).astype(np.float16)
    A[7] *= np.float16(50.0)  # one row far louder than the others
    g = rng.uniform(0.5, 1.5, K).astype(np.float16)
    _, gB, gS, _, _ = rand_case(rng, 1, K, N, 4, bs, np.float16, None)
    _, uB, uS, _, _ = rand_case(rng, 1, K, N, 4, bs, np.float16, None)
    o = ops()
    run = lambda X: host(o.matmul_nbits_mlp(dev(X), dev(gB), dev(gS), dev(uB), dev(uS), norm_scale=dev(g),
                                            block_size=bs)[0])
    Y1, Y2 = run(A), run(A)
    assert np.array_equal(Y1, Y2)
    A2 = A.copy()
    A2[7] = 0
    Y3 = run(A2)
    assert np.array_equal(np.delete(Y1, 7, 0), np.delete(Y3, 7, 0))
    ref, _ = O.matmul_nbits_mlp(A, gB, gS, uB, uS, K=K, N=N, norm_scale=g, block_size=bs)
    assert_parity(Y1, ref, np.float16)


@pytest.mark.parametrize("name", ["pinned_plain_gb_ub", "pinned_norm_nogb_noub", "pinned_skipsum_gb_ub"])
@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_fixture_mlp_pinned(gpu, name, dtype):
    case = F.find("com.microsoft.MatMulNBitsMlp", name)
    ins = F.case_inputs(case)
    conv = {k: (v.astype(dtype) if v.dtype != np.uint8 else v) for k, v in ins.items()}
    at = case["attrs"]
    Y, R = ops().matmul_nbits_mlp(dev(conv["aT"]), dev(conv["gateBT"]), dev(conv["gateScalesT"]), dev(conv["upBT"]),
                                  dev(conv["upScalesT"]), skip=dev(conv.get("skipT")),
                                  norm_scale=dev(conv.get("normScaleT")), gate_bias=dev(conv.get("gateBiasT")),
                                  up_bias=dev(conv.get("upBiasT")), block_size=at["block_size"],
                                  activation=at["activation"], want_residual=True)
    exp = F.materialize(case["outputs"]["yT"])
    if dtype == np.float32:
        assert F.reference_compare(host(Y), exp, *F.case_tolerance(case, "yT"))
        if "residualT" in case["outputs"]:
            assert F.reference_compare(host(R), F.materialize(case["outputs"]["residualT"]),
                                       *F.case_tolerance(case, "residualT"))
    else:
        ref, _ = O.matmul_nbits_mlp(conv["aT"], conv["gateBT"], conv["gateScalesT"], conv["upBT"], conv["upScalesT"],
                                    K=at["K"], N=at["N"], skip=conv.get("skipT"), norm_scale=conv.get("normScaleT"),
                                    gate_bias=conv.get("gateBiasT"), up_bias=conv.get("upBiasT"),
                                    block_size=at["block_size"])
        assert_parity(host(Y), ref, np.float16)


def test_fixture_qkv_kat(gpu):
    case = F.find("com.microsoft.MatMulNBitsQkv", "independent_nonzero_reference_qkv_kat")
    ins = F.case_inputs(case)
    Q, Kk, V, R = ops().matmul_nbits_qkv(dev(ins["aT"]), dev(ins["qBT"]), dev(ins["qScalesT"]), dev(ins["kBT"]),
                                         dev(ins["kScalesT"]), dev(ins["vBT"]), dev(ins["vScalesT"]),
                                         norm_scale=dev(ins["normScaleT"]), skip=dev(ins["skipT"]), block_size=16)
    base = 0.8320502943
    for t, c in ((Q, 1), (Kk, 2), (V, 3)):
        assert np.allclose(host(t), base * c, atol=2e-4, rtol=2e-4)
    assert np.array_equal(host(R), np.array([[1.5, 1.5, -0.75, 1.5]], np.float32))


# --------------------------------------------------------------------------- full-size workloads

def _run_workload(w):
    i, at, o = w["inputs"], w["attrs"], ops()
    d = {k: dev(v) for k, v in i.items()}
    if w["op"] == "com.microsoft.MatMulNBits":
        return [o.matmul_nbits(d["aT"], d["bT"], d["scalesT"], d.get("zeroPointsT"), d.get("biasT"),
                               block_size=at["block_size"])]
    if w["op"] == "com.microsoft.MatMulNBitsQkv":
        return list(o.matmul_nbits_qkv(d["aT"], d["qBT"], d["qScalesT"], d["kBT"], d["kScalesT"], d["vBT"],
                                       d["vScalesT"], norm_scale=d["normScaleT"], block_size=at["block_size"],
                                       epsilon=at["epsilon"], q_zero_points=d["qZeroPointsT"],
                                       k_zero_points=d["kZeroPointsT"], v_zero_points=d["vZeroPointsT"])[:3])
    return [o.matmul_nbits_mlp(d["aT"], d["gateBT"], d["gateScalesT"], d["upBT"], d["upScalesT"],
                               block_size=at["block_size"], activation=at["activation"])[0]]


def test_workload_cpu_f32_k2048(gpu):
    w = workloads.make("cpu_f32_k2048")
    i, at = w["inputs"], w["attrs"]
    y = host(_run_workload(w)[0])
    ref = O.matmul_nbits(i["aT"], i["bT"], i["scalesT"], i["zeroPointsT"], K=at["K"], N=at["N"], block_size=32)
    assert_parity(y, ref, np.float32)


def test_workload_decode_up_m1(gpu):
    w = workloads.make("decode_up_m1")
    i, at = w["inputs"], w["attrs"]
    assert ops().select_kernel("MatMulNBits", 1, at["K"], at["N"], 4, 32) == "gemv_q4_dot"
    y = host(_run_workload(w)[0])
    ref = O.matmul_nbits(i["aT"], i["bT"], i["scalesT"], K=at["K"], N=at["N"], block_size=32)
    assert_parity(y, ref, np.float16)


def test_workload_qkv_gqa_m4(gpu):
    w = workloads.make("qkv_gqa_m4")
    i, at = w["inputs"], w["attrs"]
    assert ops().select_kernel("MatMulNBitsQkv", 4, at["K"], at["Nq"], 4, at["block_size"], zp="packed") == "gemv_q4_mq"
    outs = [host(t) for t in _run_workload(w)]
    ref = O.matmul_nbits_qkv(i["aT"], i["qBT"], i["qScalesT"], i["kBT"], i["kScalesT"], i["vBT"], i["vScalesT"],
                             K=at["K"], Nq=at["Nq"], Nkv=at["Nkv"], norm_scale=i["normScaleT"],
                             block_size=at["block_size"], epsilon=at["epsilon"], q_zero_points=i["qZeroPointsT"],
                             k_zero_points=i["kZeroPointsT"], v_zero_points=i["vZeroPointsT"])
    for got, exp in zip(outs, ref[:3]):
        assert_parity(got, exp, np.float16)


def test_workload_mlp_swiglu_m16(gpu):
    w = workloads.make("mlp_swiglu_m16")
    i, at = w["inputs"], w["attrs"]
    y = host(_run_workload(w)[0])
    ref, _ = O.matmul_nbits_mlp(i["aT"], i["gateBT"], i["gateScalesT"], i["upBT"], i["upScalesT"], K=at["K"],
                                N=at["N"], block_size=at["block_size"])
    assert_parity(y, ref, np.float16)


def test_workload_prefill_m2048_row_sample(gpu):
    """Full-size prefill on the GPU; rows are independent, so a seeded sample of
    96 rows (plus the first and last) is checked against the oracle."""
    w = workloads.make("prefill_m2048")
    i, at = w["inputs"], w["attrs"]
    assert ops().select_kernel("MatMulNBits", 2048, at["K"], at["N"], 4, 128, zp="packed") == "gemm_q4_big"
    y = host(_run_workload(w)[0])
    rows = np.unique(np.concatenate([[0, 2047], np.random.default_rng(9).choice(2048, 96, replace=False)]))
    ref = O.matmul_nbits(i["aT"][rows], i["bT"], i["scalesT"], i["zeroPointsT"], i["biasT"], K=at["K"], N=at["N"],
                         block_size=at["block_size"])
    assert_parity(y[rows], ref, np.float16)
    assert np.all(np.isfinite(y))
