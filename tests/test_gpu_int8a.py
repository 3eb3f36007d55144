"""GPU: the opt-in int8-activation MatMulNBits (ops.matmul_nbits_int8a, the
upstream operator's accuracy_level 4) against its oracle (oracle/int8a.py):
seeded shapes (float32 1e-5 * max|Y|, float16 1e-2 * max|Y|), the
quantization bound against the float32 reference result, the three upstream
accuracy_level-4 cases (their fillFloat32 activations replaced by seeded
values of the same shape), and its geometry errors."""
import numpy as np
import pytest

from oracle import int8a as Q8
from oracle import oracle as O
from tests import fixture_util as F

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
MNB = "com.microsoft.MatMulNBits"


def ops():
    from xrgpu_amd import ops as _ops
    return _ops


def dev(a):
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run(A, B, S, Z, bias, K, N, bs):
    return ops().matmul_nbits_int8a(dev(A), dev(B), dev(S), dev(Z), dev(bias), K=K, N=N, block_size=bs).cpu().numpy()


CASES = [  # M, K, N, block, zero points, bias, dtype
    (1, 4096, 1000, 32, False, False, np.float16),
    (3, 4096, 257, 64, True, True, np.float32),
    (16, 1024, 128, 128, True, False, np.float16),
    (40, 512, 96, 256, False, True, np.float32),
    (2, 8192, 64, 32, True, False, np.float32),
    (8, 4096, 300, 64, True, True, np.float16),     # 32 KB of activation codes
    (9, 4096, 100, 128, False, False, np.float32),
    (64, 1024, 200, 64, True, True, np.float16),    # 64 rows
]


@pytest.mark.parametrize("M,K,N,bs,zp,bias,dt", CASES)
def test_seeded(gpu, M, K, N, bs, zp, bias, dt):
    rng = np.random.default_rng(M + K + N + bs)
    kb = K // bs
    A = (rng.standard_normal((M, K)) * rng.uniform(0.2, 4, (M, 1))).astype(dt)
    B = rng.integers(0, 256, (N, kb, bs // 2), dtype=np.uint8)
    S = rng.uniform(0.005, 0.05, (N, kb)).astype(dt)
    Z = rng.integers(0, 256, (N, (kb + 1) // 2), dtype=np.uint8) if zp else None
    b = (rng.standard_normal(N) * 0.1).astype(dt) if bias else None
    kind = O.ZP_PACKED if zp else None
    got = run(A, B, S, Z, b, K, N, bs)
    ref = Q8.matmul_nbits_int8a(A, B, S, Z, b, K=K, N=N, block_size=bs, zp_kind=kind)
    ok, err, lim = O.tolerance_ok(got, ref, dt)
    assert ok, (err, lim)
    exact = O.matmul_nbits(A, B, S, Z, b, K=K, N=N, block_size=bs, zp_kind=kind, out_dtype=np.float64)
    bound = Q8.quantization_bound(A, B, S, Z, K=K, block_size=bs, zp_kind=kind)
    slack = 1e-2 * np.abs(exact).max() if dt == np.float16 else 1e-5 * np.abs(exact).max()
    assert np.all(np.abs(got.astype(np.float64) - exact) <= bound + slack)


@pytest.mark.parametrize("name", [c["name"] for c in F.load_cases()
                                  if c["operation"] == MNB and c["attrs"].get("accuracy_level") == 4])
def test_upstream_accuracy_level4_cases(gpu, name):
    case = F.find(MNB, name)
    i = F.case_inputs(case, substitute=True)
    a = case["attrs"]
    K, N, bs = a["K"], a["N"], a.get("block_size", 32)
    A = i["aT"]
    got = run(A, i["bT"], i["scalesT"], None, None, K, N, bs)
    ref = Q8.matmul_nbits_int8a(A, i["bT"], i["scalesT"], K=K, N=N, block_size=bs)
    ok, err, lim = O.tolerance_ok(got, ref, A.dtype)
    assert ok, (err, lim)


def test_geometry_errors(gpu):
    from xrgpu_amd import _native as nat
    A = torch.zeros((1, 192), dtype=torch.float16, device="cuda")
    B = torch.zeros((8, 6, 16), dtype=torch.uint8, device="cuda")
    S = torch.ones((8, 6), dtype=torch.float16, device="cuda")
    with pytest.raises(nat.XrmmInvalid, match="K must be a positive multiple of 128|multiple of 128"):
        ops().matmul_nbits_int8a(A, B, S, K=192, N=8, block_size=32)
    A = torch.zeros((1, 256), dtype=torch.float16, device="cuda")
    B = torch.zeros((8, 16, 8), dtype=torch.uint8, device="cuda")
    S = torch.ones((8, 16), dtype=torch.float16, device="cuda")
    with pytest.raises(nat.XrmmInvalid, match="block_size"):
        ops().matmul_nbits_int8a(A, B, S, K=256, N=8, block_size=16)
