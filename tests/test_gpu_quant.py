"""GPU parity of GatherBlockQuantized and MatMulBnb4 (libxrmm through the C ABI)
against the oracle (oracle/quant.py).

GatherBlockQuantized is element-wise ((code - zero) * scale, one float32
rounding), so the bar is bit equality: every upstream case (kernels/
_provenance/upstream/com.microsoft.GatherBlockQuantized/build/webgpu/
test.json, all materialisable, two with explicit outputs), seeded tables on
both kernels (16-byte-word rows and any width), int32 / int64 indices,
duplicates, and out-of-range indices (zero rows and failure code 55).

MatMulBnb4: every upstream case (their fillFloat32 activations and absmax get
seeded stand-ins of the same shape), the reference harness's known answer
(complex_reference.py:221-250), and seeded shapes on both kernels, NF4 and FP4,
float32 (bar 1e-5 * max|Y|) and float16 (1e-2 * max|Y|).
"""
import numpy as np
import pytest

from oracle import oracle as O
from oracle import quant as Q
from tests import fixture_util as F

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
GBQ = "com.microsoft.GatherBlockQuantized"
BNB = "com.microsoft.MatMulBnb4"


def ops():
    from xrgpu_amd import ops as _ops
    return _ops


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def gbq_gpu(data, idx, scales, zps, bits, bs, **kw):
    idx = np.asarray(idx)
    it = torch.from_numpy(idx.astype(np.int64 if idx.dtype == np.int64 else np.int32)).cuda()
    return ops().gather_block_quantized(dev(data), it, dev(scales), None if zps is None else dev(zps), bits=bits,
                                        block_size=bs, **kw)


@pytest.mark.parametrize("name", [c["name"] for c in F.load_cases() if c["operation"] == GBQ])
def test_gbq_fixture_cases(gpu, name):
    case = F.find(GBQ, name)
    i = F.case_inputs(case)
    a = case["attrs"]
    bits, bs = a.get("bits", 4), a.get("block_size", 128)
    got = gbq_gpu(i["dataT"], i["indicesT"], i["scalesT"], i.get("zeroPointsT"), bits, bs).cpu().numpy()
    ref = Q.gather_block_quantized(i["dataT"], i["indicesT"], i["scalesT"], i.get("zeroPointsT"), bits=bits,
                                   block_size=bs)
    assert got.shape == ref.shape and np.array_equal(got, ref)
    if "outputT" in case["explicit"]:
        atol, rtol = F.case_tolerance(case, "outputT")
        assert F.reference_compare(got, F.materialize(case["outputs"]["outputT"]), atol, rtol)


GBQ_RAND = [  # rows, width, bits, block, zero points, int64 indices, n
    (1000, 4096, 4, 32, False, False, 64),
    (300, 4096, 4, 128, True, True, 200),
    (257, 2048, 8, 64, True, False, 33),
    (50, 72, 4, 16, True, False, 17),     # 36-byte rows: one thread per element
    (64, 1000, 8, 16, False, True, 9),    # 1000 codes: tail block of 8
]


@pytest.mark.parametrize("rows,width,bits,bs,zp,i64,n", GBQ_RAND)
def test_gbq_seeded(gpu, rows, width, bits, bs, zp, i64, n):
    rng = np.random.default_rng(rows + width + bits + bs)
    data = rng.integers(0, 256, (rows, width * bits // 8), dtype=np.uint8)
    blocks = (width + bs - 1) // bs
    scales = rng.uniform(-0.5, 0.5, (rows, blocks)).astype(np.float32)
    zps = rng.integers(0, 256, (rows, (blocks * bits + 7) // 8), dtype=np.uint8) if zp else None
    idx = rng.integers(0, rows, n).astype(np.int64 if i64 else np.int32)
    idx[: min(3, n)] = rows - 1  # duplicates and the last row
    got = gbq_gpu(data, idx, scales, zps, bits, bs).cpu().numpy()
    ref = Q.gather_block_quantized(data, idx, scales, zps, bits=bits, block_size=bs)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("width,i64", [(64, False), (72, True)])
def test_gbq_out_of_range(gpu, width, i64):
    rows = 5
    data = np.arange(rows * width // 2, dtype=np.uint8).reshape(rows, width // 2)
    scales = np.full((rows, (width + 15) // 16), 0.5, np.float32)
    idx = np.array([1, rows, -1, 2] + ([2 ** 40] if i64 else []), np.int64 if i64 else np.int32)
    with pytest.raises(Exception, match="code 55"):
        gbq_gpu(data, idx, scales, None, 4, 16)
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    got = gbq_gpu(data, idx, scales, None, 4, 16, status=status, check=False).cpu().numpy()
    assert int(status.item()) == 55
    ref = Q.gather_block_quantized(data, idx, scales, None, bits=4, block_size=16, strict=False)
    assert np.array_equal(got, ref)
    assert np.all(got[1] == 0) and np.all(got[2] == 0)


def bnb_gpu(a, b, absmax, K, N, bs, qt, tb=1):
    return ops().matmul_bnb4(dev(a), dev(b), dev(absmax), K=K, N=N, block_size=bs, quant_type=qt,
                             trans_b=tb).cpu().numpy()


def bnb_check(got, ref, dtype):
    ok, err, lim = O.tolerance_ok(got, ref, dtype)
    assert ok, f"max|d|={err} > {lim}"


@pytest.mark.parametrize("name", [c["name"] for c in F.load_cases() if c["operation"] == BNB])
def test_bnb4_fixture_cases(gpu, name):
    case = F.find(BNB, name)
    i = F.case_inputs(case, substitute=True)
    a = case["attrs"]
    K, N = a["K"], a["N"]
    bs, qt, tb = a.get("block_size", 32), a.get("quant_type", 1), a.get("transB", 1)
    got = bnb_gpu(i["aT"], i["bT"], i["absmaxT"], K, N, bs, qt, tb)
    ref = Q.matmul_bnb4(i["aT"], i["bT"], i["absmaxT"], K=K, N=N, block_size=bs, quant_type=qt, trans_b=tb)
    assert got.shape == ref.shape
    bnb_check(got, ref, i["aT"].dtype)


def test_bnb4_reference_known_answer(gpu):
    a = np.array([[1, -2, 0.5, 3]], np.float32)
    packed = np.array([240, 120, 105, 171], np.uint8)
    got = bnb_gpu(a, packed, np.array([1], np.float32), 4, 2, 16, 1)
    ref = Q.matmul_bnb4(a, packed, np.array([1], np.float32), K=4, N=2, block_size=16, quant_type=1)
    assert np.allclose(got, ref, rtol=0, atol=1e-6)


BNB_RAND = [  # M, K, N, block, quant_type, dtype, transB, kernel
    (1, 4096, 1000, 64, 1, np.float16, 1, "bnb4_gemv"),
    (1, 2048, 333, 32, 0, np.float32, 1, "bnb4_gemv"),
    (2, 1024, 257, 16, 1, np.float32, 1, "bnb4_gemv"),
    (3, 4096, 96, 128, 0, np.float16, 1, "bnb4_gemv"),
    (7, 512, 64, 256, 1, np.float32, 1, "bnb4_gemv"),
    (16, 2048, 130, 16, 0, np.float16, 1, "bnb4_gemv"),
    (4, 96, 40, 48, 1, np.float32, 1, "bnb4_scalar"),    # blocks of 48 straddle 32-code chunks
    (2, 64, 24, 16, 0, np.float16, 0, "bnb4_scalar"),    # transB = 0
    (3, 33, 19, 16, 1, np.float32, 1, "bnb4_scalar"),    # K not a multiple of 32
]


@pytest.mark.parametrize("M,K,N,bs,qt,dt,tb,kernel", BNB_RAND)
def test_bnb4_seeded(gpu, M, K, N, bs, qt, dt, tb, kernel):
    rng = np.random.default_rng(M * 7 + K + N + bs)
    a = rng.standard_normal((M, K)).astype(dt)
    b = rng.integers(0, 256, (N * K + 1) // 2, dtype=np.uint8)
    absmax = rng.uniform(0.05, 1.5, (N * K + bs - 1) // bs).astype(dt)
    assert ops().bnb4_kernel(M, K, N, bs, qt, tb, torch.float16 if dt == np.float16 else torch.float32) == kernel
    got = bnb_gpu(a, b, absmax, K, N, bs, qt, tb)
    ref = Q.matmul_bnb4(a, b, absmax, K=K, N=N, block_size=bs, quant_type=qt, trans_b=tb)
    bnb_check(got, ref, dt)
