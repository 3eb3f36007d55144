"""Pins for the CPU oracle (no GPU). Every oracle function is checked against a
golden vector from the reference, a closed form or an independent brute force."""
import numpy as np
import pytest

from oracle import oracle as O
from oracle import serial
from tests import fixture_util as F
from xrgpu_amd import workloads

MNB = "com.microsoft.MatMulNBits"
MLP = "com.microsoft.MatMulNBitsMlp"
QKV = "com.microsoft.MatMulNBitsQkv"


def bitstring_codes(B, K, bits, block_size):
    """Independent brute force: each blob is a little-endian bit string and
    code e of a block occupies bits [e*bits, (e+1)*bits)."""
    N, kb, blob = B.shape
    out = np.zeros((N, K), np.int64)
    for n in range(N):
        for b in range(kb):
            bitsarr = np.unpackbits(B[n, b], bitorder="little")
            for e in range(block_size):
                k = b * block_size + e
                if k >= K:
                    break
                word = bitsarr[e * bits:(e + 1) * bits]
                out[n, k] = int(sum(int(v) << i for i, v in enumerate(word)))
    return out


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_unpack_every_byte_value(bits):
    # all 256 byte values at every element offset of a block
    per = 8 // bits
    bs = 16
    blob = O.blob_bytes(bs, bits)
    vals = np.arange(256, dtype=np.uint8)
    B = np.zeros((256, 1, blob), np.uint8)
    B[:, 0, :] = vals[:, None]
    codes = O.unpack_codes(B, bs, bits, bs)
    for v in range(256):
        expect = [(v >> (bits * i)) & ((1 << bits) - 1) for i in range(per)] * (bs // per)
        assert list(codes[v]) == expect


@pytest.mark.parametrize("bits,bs,K", [(4, 32, 70), (2, 16, 33), (8, 16, 40), (4, 8, 16), (4, 16, 17)])
def test_unpack_matches_bitstring_brute_force(bits, bs, K):
    rng = np.random.default_rng(bits * 100 + bs + K)
    kb = O.k_blocks(K, bs)
    B = rng.integers(0, 256, size=(3, kb, O.blob_bytes(bs, bits)), dtype=np.uint8)
    assert np.array_equal(O.unpack_codes(B, K, bits, bs), bitstring_codes(B, K, bits, bs))


def test_unpack_qkv_kat_bytes():
    # complex_reference.py:251-272: bytes 152/168/184 give weights [0,c,0,c]*0.5
    for byte, hi in ((152, 9), (168, 10), (184, 11)):
        B = np.full((2, 1, 8), byte, np.uint8)
        q = O.unpack_codes(B, 4, 4, 16)
        assert list(q[0]) == [8, hi, 8, hi]
        W = O.dequantize(B, np.full((2, 1), 0.5, np.float32), None, 4, 4, 16)
        assert list(W[1]) == [0.0, (hi - 8) * 0.5, 0.0, (hi - 8) * 0.5]


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_packed_zero_points_bit_order(bits):
    rng = np.random.default_rng(bits)
    kb = 13
    zp = rng.integers(0, 256, size=(5, O.packed_zp_bytes(kb, bits)), dtype=np.uint8)
    got = O.unpack_packed_zero_points(zp, kb, bits)
    want = bitstring_codes(zp[:, None, :], kb, bits, kb)  # one "block" holding kb codes
    assert np.array_equal(got, want)


@pytest.mark.parametrize("bits,bs", [(4, 32), (2, 16), (8, 32), (4, 128)])
def test_packed_zero_points_equal_float_zero_points(bits, bs):
    """Invariant pinning the packed-zp extension to reference semantics: the
    packed form gives the same result as float zero points holding the
    unpacked values (float zp is the reference's own path)."""
    rng = np.random.default_rng(7 + bits)
    K, N = 3 * bs + 5, 6
    kb = O.k_blocks(K, bs)
    A = rng.standard_normal((3, K)).astype(np.float32)
    B = rng.integers(0, 256, size=(N, kb, O.blob_bytes(bs, bits)), dtype=np.uint8)
    S = rng.uniform(0.001, 0.02, (N, kb)).astype(np.float32)
    zp = rng.integers(0, 256, size=(N, O.packed_zp_bytes(kb, bits)), dtype=np.uint8)
    zf = O.unpack_packed_zero_points(zp, kb, bits).astype(np.float32)
    y1 = O.matmul_nbits(A, B, S, zp, K=K, N=N, bits=bits, block_size=bs)
    y2 = O.matmul_nbits(A, B, S, zf, K=K, N=N, bits=bits, block_size=bs)
    assert np.array_equal(y1, y2)
    ys = serial.matmul_nbits(A, B, S, zf, K=K, N=N, bits=bits, block_size=bs)
    assert O.tolerance_ok(ys, y1, np.float32)[0]


def test_dequantize_closed_form_exact():
    # (code - z) * scale with a power-of-two scale is exact in float32 and float16
    B = np.array([[[0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE]]], np.uint8)
    W = O.dequantize(B, np.array([[0.25]], np.float32), None, 16, 4, 16)
    assert list(W[0]) == [(c - 8) * 0.25 for c in range(16)]
    zf = np.array([[3.0]], np.float32)
    W = O.dequantize(B, np.array([[2.0]], np.float16), zf, 16, 4, 16, stage="f16")
    assert W.dtype == np.float16 and list(W[0].astype(np.float32)) == [(c - 3) * 2.0 for c in range(16)]


def test_dequantize_f16_stage_is_one_rounding_of_f32():
    rng = np.random.default_rng(3)
    B = rng.integers(0, 256, size=(64, 4, 16), dtype=np.uint8)
    S = rng.uniform(1e-7, 2.0, (64, 4)).astype(np.float16)  # includes f16 subnormal products
    zp = rng.integers(0, 256, size=(64, 2), dtype=np.uint8)
    w32 = O.dequantize(B, S, zp, 128, 4, 32)
    w16 = O.dequantize(B, S, zp, 128, 4, 32, stage="f16")
    # integer (code - z) times an fp16 scale is exact in float32, so the fp16
    # stage equals the correctly rounded exact product
    exact = (O.unpack_codes(B, 128, 4, 32).astype(np.float64)
             - O.unpack_packed_zero_points(zp, 4, 4).astype(np.float64)[:, np.arange(128) // 32]) \
        * S.astype(np.float64)[:, np.arange(128) // 32]
    assert np.array_equal(w32.astype(np.float64), exact)
    assert np.array_equal(w16, exact.astype(np.float16))


def test_fixture_block512_exact():
    case = F.find(MNB, "q4_block512_schema_legal_cpu_provider_gap_exact")
    ins = F.case_inputs(case)
    at = case["attrs"]
    y = O.matmul_nbits(ins["aT"], ins["bT"], ins["scalesT"], K=at["K"], N=at["N"], bits=at["bits"],
                       block_size=at["block_size"])
    expected = F.materialize(case["outputs"]["yT"])
    assert np.array_equal(y, expected) and y[0, 0] == 128.0
    ys = serial.matmul_nbits(ins["aT"], ins["bT"], ins["scalesT"], K=512, N=1, bits=4, block_size=512)
    assert ys[0, 0] == 128.0


@pytest.mark.parametrize("name", ["empty_zero_dim", "empty_zero_dim_f16"])
def test_fixture_empty_m(name):
    case = F.find(MNB, name)
    ins = F.case_inputs(case)
    at = case["attrs"]
    y = O.matmul_nbits(ins["aT"], ins["bT"], ins["scalesT"], K=at["K"], N=at["N"], bits=4, block_size=32)
    exp = F.materialize(case["outputs"]["yT"])
    assert y.shape == exp.shape == (0, 4) and y.dtype == exp.dtype


@pytest.mark.parametrize("name", ["ort_f16_large_k_accumulator_cancellation_m1_k8192_n8",
                                  "ort_f16_large_k_accumulator_cancellation_m8_k8192_n8",
                                  "f16_full_k_accumulator_cancellation_prefill_m64_k4096_n64"])
def test_fixture_accumulator_cancellation(name):
    # provenance notes: exact result 0 while partial sums exceed the fp16 range
    case = F.find(MNB, name)
    ins = F.case_inputs(case)
    at = case["attrs"]
    y = O.matmul_nbits(ins["aT"], ins["bT"], ins["scalesT"], K=at["K"], N=at["N"], bits=4, block_size=32)
    assert y.dtype == np.float16 and np.all(y == 0)
    atol, rtol = F.case_tolerance(case, "yT")
    assert F.reference_compare(y, np.zeros_like(y), atol, rtol)


@pytest.mark.parametrize("name", ["pinned_plain_gb_ub", "pinned_norm_nogb_noub", "pinned_skipsum_gb_ub"])
def test_fixture_mlp_pinned(name):
    case = F.find(MLP, name)
    ins = F.case_inputs(case)
    at = case["attrs"]
    y, r = O.matmul_nbits_mlp(ins["aT"], ins["gateBT"], ins["gateScalesT"], ins["upBT"], ins["upScalesT"],
                              K=at["K"], N=at["N"], skip=ins.get("skipT"), norm_scale=ins.get("normScaleT"),
                              gate_bias=ins.get("gateBiasT"), up_bias=ins.get("upBiasT"), bits=at["bits"],
                              block_size=at["block_size"], activation=at["activation"])
    atol, rtol = F.case_tolerance(case, "yT")
    assert F.reference_compare(y, F.materialize(case["outputs"]["yT"]), atol, rtol)
    if "residualT" in case["outputs"]:
        atol, rtol = F.case_tolerance(case, "residualT")
        assert F.reference_compare(r, F.materialize(case["outputs"]["residualT"]), atol, rtol)
    ys, rs = serial.matmul_nbits_mlp(ins["aT"], ins["gateBT"], ins["gateScalesT"], ins["upBT"], ins["upScalesT"],
                                     K=at["K"], N=at["N"], skip=ins.get("skipT"), norm_scale=ins.get("normScaleT"),
                                     gate_bias=ins.get("gateBiasT"), up_bias=ins.get("upBiasT"),
                                     bits=at["bits"], block_size=at["block_size"])
    assert F.reference_compare(ys, F.materialize(case["outputs"]["yT"]), *F.case_tolerance(case, "yT"))


def test_fixture_qkv_kat():
    case = F.find(QKV, "independent_nonzero_reference_qkv_kat")
    ins = F.case_inputs(case)
    q, k, v, r = O.matmul_nbits_qkv(ins["aT"], ins["qBT"], ins["qScalesT"], ins["kBT"], ins["kScalesT"],
                                    ins["vBT"], ins["vScalesT"], K=4, Nq=2, Nkv=2, norm_scale=ins["normScaleT"],
                                    skip=ins["skipT"], block_size=16)
    # hand-derived: r=[1.5,1.5,-.75,1.5], mean(r^2)=1.828125, x=r/sqrt(1.828126)*gamma,
    # projections pick x[1]+x[3] times (code-8)*0.5
    x = np.array([1.5, 1.5 * 0.5, -0.75 * 2, 1.5]) / np.sqrt(1.828125 + 1e-6)
    base = (x[1] + x[3]) * 0.5
    for out, c in ((q, 1), (k, 2), (v, 3)):
        assert np.allclose(out, base * c, atol=2e-4, rtol=2e-4)
    assert np.allclose(base, 0.8320502943, atol=1e-6)
    assert np.array_equal(r, np.array([[1.5, 1.5, -0.75, 1.5]], np.float32))


def test_qkv_equals_three_matmuls_on_normalised_input():
    rng = np.random.default_rng(11)
    K, Nq, Nkv, bs = 128, 32, 16, 64
    kb = K // bs
    A = rng.standard_normal((3, K)).astype(np.float16)
    skip = rng.standard_normal((3, K)).astype(np.float16)
    g = rng.uniform(0.5, 1.5, K).astype(np.float16)
    Bs = [rng.integers(0, 256, (n, kb, bs // 2), dtype=np.uint8) for n in (Nq, Nkv, Nkv)]
    Ss = [rng.uniform(.001, .02, (n, kb)).astype(np.float16) for n in (Nq, Nkv, Nkv)]
    Zs = [rng.integers(0, 256, (n, 1), dtype=np.uint8) for n in (Nq, Nkv, Nkv)]
    q, k, v, r = O.matmul_nbits_qkv(A, Bs[0], Ss[0], Bs[1], Ss[1], Bs[2], Ss[2], K=K, Nq=Nq, Nkv=Nkv,
                                    norm_scale=g, skip=skip, block_size=bs, q_zero_points=Zs[0],
                                    k_zero_points=Zs[1], v_zero_points=Zs[2], out_dtype=np.float32)
    x, _ = O.normalized_input(A, K, skip, g, 1e-6)
    for out, Bm, S, Z, n in zip((q, k, v), Bs, Ss, Zs, (Nq, Nkv, Nkv)):
        ref = O.matmul_nbits(x, Bm, S, Z, K=K, N=n, block_size=bs, out_dtype=np.float32)
        assert np.allclose(out, ref, rtol=1e-6, atol=1e-6)
    # the serial float32 order of the reference agrees far inside the fp32 bar
    sq, sk_, sv, sr = serial.matmul_nbits_qkv(A, Bs, Ss, K=K, Nq=Nq, Nkv=Nkv, norm_scale=g, skip=skip,
                                              zero_points=Zs, block_size=bs)
    for a_, b_ in ((sq, q), (sk_, k), (sv, v)):
        assert O.tolerance_ok(a_, b_, np.float32)[0]
    assert np.array_equal(sr, r.astype(np.float32))


def test_activation_closed_forms():
    x = np.array([-3.0, -0.5, 0.0, 0.5, 3.0])
    assert np.array_equal(O.fused_activation(x, 1), np.maximum(x, 0))
    assert np.allclose(O.fused_activation(x, 5), 1 / (1 + np.exp(-x)))
    assert np.allclose(O.fused_activation(x, 2), x / (1 + np.exp(-x)))
    assert np.allclose(O.fused_activation(x, 4), np.tanh(x))
    assert np.array_equal(O.fused_activation(x, 0), x)
    # large negative inputs stay finite (the guarded logistic form)
    assert O.fused_activation(np.array([-1000.0]), 2)[0] == 0.0


def _reference_erf(x):
    """The reference shader's own erf (complex_math.glsl:185-199): an odd Taylor
    series below 0.5, sign(x) above 6, Abramowitz and Stegun 7.1.26 between
    (absolute error <= 1.5e-7). An approximation independent of scipy's erf,
    so agreement pins the oracle's gelu to the erf form the shader evaluates."""
    x = np.asarray(x, dtype=np.float64)
    t = np.abs(x)
    z = x * x
    p = 1.0 + z * (-1 / 3 + z * (1 / 10 + z * (-1 / 42 + z * (1 / 216 + z * (-1 / 1320 + z * (1 / 9360 - z / 75600))))))
    small = 1.1283791670955126 * x * p
    a = 1.0 / (1.0 + 0.3275911 * t)
    q = (((((1.061405429 * a - 1.453152027) * a) + 1.421413741) * a - 0.284496736) * a + 0.254829592) * a
    y = np.sign(x) * (1.0 - q * np.exp(-t * t))
    return np.where(t < 0.5, small, np.where(t > 6.0, np.sign(x), y))


def test_gelu_is_the_erf_form():
    """fused kind 3 for opcode 1027 is 0.5 x (1 + erf(x / sqrt 2))
    (complex_kernel.glsl:41-44), not the tanh form the other opcodes use."""
    g = lambda v: float(O.fused_activation(np.array([v]), 3)[0])  # noqa: E731
    # x * Phi(x) at +-1: Phi(1) = 0.8413447460685429 (standard normal CDF)
    assert abs(g(1.0) - 0.8413447460685429) < 1e-15
    assert abs(g(-1.0) - (-0.15865525393145707)) < 1e-15
    assert g(0.0) == 0.0
    # erf is odd, so gelu(x) - gelu(-x) = x exactly in real arithmetic
    x = np.linspace(-8.0, 8.0, 321)
    d = O.fused_activation(x, 3) - O.fused_activation(-x, 3)
    assert np.allclose(d, x, rtol=0, atol=1e-14)
    # far from the tanh approximation where the two forms part (|x| near 2.5-3)
    tanh_form = 0.5 * x * (1 + np.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3)))
    for v in (2.5, -2.5, 3.0, -3.0):
        i = int(np.argmin(np.abs(x - v)))
        assert abs(O.fused_activation(x[i:i + 1], 3)[0] - tanh_form[i]) > 1e-4
    # and within the shader's own erf approximation's bound everywhere
    ref = 0.5 * x * (1.0 + _reference_erf(x * 0.7071067811865475))
    assert np.max(np.abs(O.fused_activation(x, 3) - ref) / np.maximum(np.abs(x), 1.0)) < 2e-7


def test_gelu_serial_float32_order_matches():
    """The serial float32 restatement (erff) of the gelu Mlp path agrees with
    the float64 oracle within the fp32 bar."""
    rng = np.random.default_rng(33)
    M, K, N, bs = 3, 96, 7, 32
    kb = O.k_blocks(K, bs)
    A = rng.standard_normal((M, K)).astype(np.float32)
    gB, uB = (rng.integers(0, 256, (N, kb, bs // 2), dtype=np.uint8) for _ in range(2))
    gS, uS = (rng.uniform(0.01, 0.2, (N, kb)).astype(np.float32) for _ in range(2))
    gb = rng.standard_normal(N).astype(np.float32)
    y, _ = O.matmul_nbits_mlp(A, gB, gS, uB, uS, K=K, N=N, gate_bias=gb, block_size=bs, activation="gelu")
    ys, _ = serial.matmul_nbits_mlp(A, gB, gS, uB, uS, K=K, N=N, gate_bias=gb, block_size=bs, act=3)
    ok, err, lim = O.tolerance_ok(ys, y, np.float32)
    assert ok, (err, lim)
    # the gelu result differs from the silu one (the activation kind reaches the epilogue)
    ysilu, _ = O.matmul_nbits_mlp(A, gB, gS, uB, uS, K=K, N=N, gate_bias=gb, block_size=bs, activation="silu")
    assert not O.tolerance_ok(ysilu, y, np.float32)[0]


@pytest.mark.parametrize("bits,bs,K,N,M,zp", [(4, 32, 70, 5, 3, "packed"), (2, 16, 33, 4, 2, "float"),
                                             (8, 16, 40, 3, 1, "none"), (4, 128, 256, 9, 2, "float")])
def test_numpy_oracle_matches_serial_float32_order(bits, bs, K, N, M, zp):
    rng = np.random.default_rng(K + N)
    kb = O.k_blocks(K, bs)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.integers(0, 256, size=(N, kb, O.blob_bytes(bs, bits)), dtype=np.uint8)
    S = rng.uniform(0.001, 0.02, (N, kb)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    Z = None
    if zp == "packed":
        Z = rng.integers(0, 256, size=(N, O.packed_zp_bytes(kb, bits)), dtype=np.uint8)
    elif zp == "float":
        Z = rng.uniform(0, (1 << bits) - 1, (N, kb)).astype(np.float32)
    y = O.matmul_nbits(A, B, S, Z, bias, K=K, N=N, bits=bits, block_size=bs)
    ys = serial.matmul_nbits(A, B, S, Z, bias, K=K, N=N, bits=bits, block_size=bs)
    ok, err, lim = O.tolerance_ok(ys, y, np.float32)
    assert ok, (err, lim)


def test_cpu_workload_fp32_bar_against_serial_order():
    """The CPU-runnable workload (K=N=2048, f32, packed zp, seed 0): the float64
    oracle and the reference's serial float32 order agree within 1e-5*max|Y|."""
    w = workloads.make("cpu_f32_k2048")
    i, at = w["inputs"], w["attrs"]
    y = O.matmul_nbits(i["aT"], i["bT"], i["scalesT"], i["zeroPointsT"], K=at["K"], N=at["N"], block_size=32)
    ys = serial.matmul_nbits(i["aT"], i["bT"], i["scalesT"], i["zeroPointsT"], K=at["K"], N=at["N"], block_size=32)
    ok, err, lim = O.tolerance_ok(ys, y, np.float32)
    assert ok and np.all(np.isfinite(y)), (err, lim)


def test_tolerance_rule():
    e = np.array([1.0, -2.0, 0.5], np.float16)
    assert O.tolerance_ok(e + np.float16(0.015), e, np.float16)[0]
    assert not O.tolerance_ok(e + np.float16(0.03), e, np.float16)[0]
    assert not O.tolerance_ok(np.array([np.nan, 0, 0]), np.zeros(3), np.float16)[0]


def test_tolerance_rule_nonfinite():
    inf, nan = np.inf, np.nan
    e = np.array([inf, -inf, nan, 1.0])
    assert O.tolerance_ok(np.array([inf, -inf, nan, 1.0]), e, np.float32)[0]
    assert not O.tolerance_ok(np.array([-inf, -inf, nan, 1.0]), e, np.float32)[0]  # sign of Inf
    assert not O.tolerance_ok(np.array([inf, -inf, 0.0, 1.0]), e, np.float32)[0]   # NaN expected
    assert not O.tolerance_ok(np.array([inf, nan, nan, 1.0]), e, np.float32)[0]    # Inf expected


def nonfinite_activations(rng, M, K, dtype):
    """Rows with +Inf, -Inf, both (columns may cancel to NaN), NaN, then finite rows."""
    A = rng.standard_normal((M, K)).astype(dtype)
    pos = rng.permutation(K)[:4]
    if M > 0:
        A[0, pos[0]] = np.inf
    if M > 1:
        A[1, pos[1]] = -np.inf
    if M > 2:
        A[2, pos[2]], A[2, pos[3]] = np.inf, -np.inf
    if M > 3:
        A[3, pos[0]] = np.nan
    return A


@pytest.mark.parametrize("zp", ["none", "packed", "float"])
def test_nonfinite_policy_matches_serial_order(zp):
    """+-Inf / NaN activations: the float64 oracle gives the same non-finite
    pattern (NaN, +Inf, -Inf per element) as the reference's serial float32
    loop ``sum += a * W`` (complex_kernel.glsl:83) restated in C, and the same
    finite values within the fp32 bar. Codes equal to the zero point make
    W = 0, so Inf * 0 = NaN cases occur."""
    rng = np.random.default_rng(71)
    M, K, N, bs = 5, 96, 40, 32
    kb = O.k_blocks(K, bs)
    A = nonfinite_activations(rng, M, K, np.float32)
    B = rng.integers(0, 256, (N, kb, bs // 2), dtype=np.uint8)
    S = rng.uniform(0.01, 0.2, (N, kb)).astype(np.float32)
    Z = None
    if zp == "packed":
        Z = rng.integers(0, 256, (N, O.packed_zp_bytes(kb, 4)), dtype=np.uint8)
    elif zp == "float":
        Z = rng.integers(0, 16, (N, kb)).astype(np.float32)
    y = O.matmul_nbits(A, B, S, Z, K=K, N=N, block_size=bs)
    ys = serial.matmul_nbits(A, B, S, Z, K=K, N=N, block_size=bs)
    for f in (np.isnan, np.isposinf, np.isneginf):
        assert np.array_equal(f(y), f(ys))
    assert np.isnan(y).any() and np.isposinf(y).any() and np.isneginf(y).any()
    assert np.all(np.isfinite(y[4:]))
    assert O.tolerance_ok(ys, y, np.float32)[0]


@pytest.mark.parametrize("N,K,bs", [(37, 96, 32), (5, 20, 16), (16, 256, 128), (3, 4096, 64), (7, 200, 32)])
def test_prepack_layout_decodes_to_the_codes(N, K, bs):
    """The prefill GEMM's prepacked layout, decoded the way the GEMM reads it
    (per word, exponent-bias pairs from nibble slots 0/4, 1/5, 2/6, 3/7 in
    k order; K step s of column n at bytes (s N + n) 32 .. + 31), gives back
    oracle.unpack_codes; the padding half past the last chunk is zero."""
    from oracle import prepack as PK
    rng = np.random.default_rng(N * 7 + K + bs)
    kb = O.k_blocks(K, bs)
    B = rng.integers(0, 256, size=(N, kb, O.blob_bytes(bs, 4)), dtype=np.uint8)
    flat = PK.prepack_q4(B, K, bs)
    assert flat.size == PK.packed_bytes(N, K, bs)
    Kp = kb * bs
    ksteps = (Kp + 63) // 64
    codes = np.zeros((N, ksteps * 64), dtype=np.uint8)
    for s in range(ksteps):
        for n in range(N):
            piece = flat[(s * N + n) * 32:(s * N + n) * 32 + 32]
            for w in range(8):
                word = int.from_bytes(bytes(piece[4 * w:4 * w + 4]), "little")
                slots = [(word >> (4 * j)) & 15 for j in range(8)]
                for pair in range(4):  # the GEMM's pair p yields k = 2p, 2p + 1
                    codes[n, s * 64 + 8 * w + 2 * pair] = slots[pair]
                    codes[n, s * 64 + 8 * w + 2 * pair + 1] = slots[pair + 4]
    assert np.array_equal(codes[:, :K], O.unpack_codes(B, K, 4, bs))
    assert not codes[:, Kp:].any()  # the zero half past the last chunk
    assert PK.packed_bytes(N, K, bs, bits=8) == 0
