"""Pins of the GatherBlockQuantized / MatMulBnb4 oracle (oracle/quant.py), CPU.

GatherBlockQuantized:
* the two explicit upstream outputs (kernels/_provenance/upstream/
  com.microsoft.GatherBlockQuantized/build/webgpu/test.json: the 8-bit
  default-midpoint case and the 4-bit zero-point case with a tail block);
* every other upstream case (all materialisable) runs with the right shape;
* equality with the independently pinned MatMulNBits dequantisation
  (oracle.dequantize, same low-first codes and packed zero points) on the
  gathered rows;
* out-of-range indices fail (code 55) and leave zero rows; int64 indices
  saturate to int32 as controlIndex does.

MatMulBnb4:
* the NF4 codebook against its published construction (normal quantiles with
  offset 0.9677083, bitsandbytes' create_normal_map) and the FP4 codebook
  against its sign / 2-bit exponent / 1-bit mantissa construction;
* the reference harness's known answer (kernels/_shared/extended/
  complex_reference.py:221-250: bytes 240 120 105 171, K=4, N=2, NF4), whose
  expectation is formed here from the constructed codebook and codes read off
  the bytes by hand (high nibble first);
* the flat-index layout (transB 1 and 0, blocks straddling rows when
  K % block_size != 0) against dequantising the flat array and reshaping it.
"""
import numpy as np
import pytest
from scipy.stats import norm

from oracle import oracle as O
from oracle import quant as Q
from tests import fixture_util as F

GBQ = "com.microsoft.GatherBlockQuantized"


def gbq_case(case):
    i = F.case_inputs(case)
    a = case["attrs"]
    return Q.gather_block_quantized(i["dataT"], i["indicesT"], i["scalesT"], i.get("zeroPointsT"),
                                    bits=a.get("bits", 4), block_size=a.get("block_size", 128))


@pytest.mark.parametrize("name", ["ort_q8_no_zero_points_default_midpoint",
                                  "ort_projection_q4_zero_points_block16_tail_rows"])
def test_gbq_explicit_outputs(name):
    case = F.find(GBQ, name)
    want = F.materialize(case["outputs"]["outputT"])
    got = gbq_case(case)
    atol, rtol = F.case_tolerance(case, "outputT")
    assert got.shape == want.shape and F.reference_compare(got, want, atol, rtol)


@pytest.mark.parametrize("name", [c["name"] for c in F.load_cases() if c["operation"] == GBQ])
def test_gbq_all_cases_shapes(name):
    case = F.find(GBQ, name)
    got = gbq_case(case)
    assert got.shape == tuple(case["outputs"]["outputT"]["shape"])
    assert got.dtype == np.float32


@pytest.mark.parametrize("bits,block,zp", [(4, 16, False), (4, 32, True), (8, 16, True), (8, 64, False)])
def test_gbq_equals_matmul_nbits_dequantisation(bits, block, zp):
    rng = np.random.default_rng(bits * 100 + block + zp)
    rows, width = 7, 128
    data = rng.integers(0, 256, (rows, width * bits // 8), dtype=np.uint8)
    kb = width // block
    scales = rng.uniform(0.01, 0.5, (rows, kb)).astype(np.float32)
    zps = rng.integers(0, 256, (rows, (kb * bits + 7) // 8), dtype=np.uint8) if zp else None
    idx = np.array([6, 0, 3, 3, 1], np.int32)
    got = Q.gather_block_quantized(data, idx, scales, zps, bits=bits, block_size=block)
    W = O.dequantize(data.reshape(rows, kb, block * bits // 8), scales, zps, width, bits, block,
                     zp_kind=O.ZP_PACKED if zp else None)
    assert np.array_equal(got, W[idx])


def test_gbq_index_failures_and_int64():
    data = np.arange(32, dtype=np.uint8).reshape(4, 8)
    scales = np.ones((4, 1), np.float32)
    with pytest.raises(Q.GatherIndexError):
        Q.gather_block_quantized(data, np.array([0, 4], np.int32), scales, bits=4, block_size=16)
    out = Q.gather_block_quantized(data, np.array([1, -1, 2], np.int32), scales, bits=4, block_size=16, strict=False)
    assert np.all(out[1] == 0) and np.any(out[0] != 0) and np.any(out[2] != 0)
    big = np.array([2 ** 33, -(2 ** 40), 3], np.int64)
    assert list(Q.control_index(big)) == [2 ** 31 - 1, -(2 ** 31), 3]
    out = Q.gather_block_quantized(data, big, scales, bits=4, block_size=16, strict=False)
    assert np.all(out[:2] == 0) and np.array_equal(out[2], Q.gather_block_quantized(data, [3], scales, bits=4,
                                                                                     block_size=16)[0])


def constructed_nf4():
    offset = 0.9677083
    pos = norm.ppf(np.linspace(offset, 0.5, 9)[:-1])
    neg = -norm.ppf(np.linspace(offset, 0.5, 8)[:-1])
    v = np.sort(np.concatenate([pos, [0.0], neg]))
    return v / v.max()


def constructed_fp4():
    # code = sign(bit 3) | exponent field (bits 2..1) | mantissa (bit 0);
    # field 0 is subnormal (m/16), fields 1..3 are (1 + m/2) * 2^(4 - field);
    # values normalised by the largest (12)
    out = []
    for c in range(16):
        s, e, m = c >> 3, (c >> 1) & 3, c & 1
        mag = m / 16 if e == 0 else (1 + m / 2) * 2.0 ** (4 - e)
        out.append((-1) ** s * mag / 12)
    return np.array(out)


def test_codebooks_match_their_construction():
    assert np.max(np.abs(Q.NF4.astype(np.float64) - constructed_nf4())) < 2e-7
    assert np.max(np.abs(Q.FP4.astype(np.float64) - constructed_fp4())) < 1e-15 + 1e-7
    assert np.signbit(Q.FP4[8]) and Q.FP4[8] == 0


def test_bnb4_reference_known_answer():
    a = np.array([[1, -2, 0.5, 3]], np.float32)
    packed = np.array([240, 120, 105, 171], np.uint8)
    # high nibble first: 0xF0 -> 15, 0; 0x78 -> 7, 8; 0x69 -> 6, 9; 0xAB -> 10, 11
    codes = [[15, 0, 7, 8], [6, 9, 10, 11]]
    book = constructed_nf4()
    want = np.array([[sum(a[0, k] * book[codes[n][k]] for k in range(4)) for n in range(2)]])
    got = Q.matmul_bnb4(a, packed, np.array([1], np.float32), K=4, N=2, block_size=16, quant_type=1)
    assert np.allclose(got, want, rtol=0, atol=1e-6)


@pytest.mark.parametrize("K,N,bs,qt,tb", [(33, 19, 16, 1, 1), (64, 24, 32, 0, 1), (40, 12, 16, 1, 0), (48, 8, 64, 0, 0)])
def test_bnb4_flat_layout(K, N, bs, qt, tb):
    rng = np.random.default_rng(K * N + bs)
    b = rng.integers(0, 256, (K * N + 1) // 2, dtype=np.uint8)
    absmax = rng.uniform(0.1, 2.0, (K * N + bs - 1) // bs).astype(np.float32)
    # independent route: dequantise the flat stream, then reshape it
    hi, lo = b >> 4, b & 15
    codes = np.stack([hi, lo], axis=1).reshape(-1)[:K * N]
    book = Q.NF4 if qt == 1 else Q.FP4
    flat = book[codes] * np.repeat(absmax, bs)[:K * N]
    W = flat.reshape(N, K).T if tb else flat.reshape(K, N)
    assert np.array_equal(Q.bnb_weights(b, absmax, K, N, bs, qt, tb), W.astype(np.float32))
    a = rng.standard_normal((3, K)).astype(np.float32)
    got = Q.matmul_bnb4(a, b, absmax, K=K, N=N, block_size=bs, quant_type=qt, trans_b=tb)
    assert np.allclose(got, (a.astype(np.float64) @ W.astype(np.float64)).astype(np.float32), rtol=1e-6, atol=1e-6)
