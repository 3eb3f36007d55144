"""The prefill GEMM on prepacked weights (xrmm_prepack_weights,
xrmm_matmul_nbits_prepacked) against the oracle.

Bars: the device prepack is bit-exact against oracle/prepack.py (itself pinned
to oracle.unpack_codes); the GEMM on the prepacked layout meets the float16 bar
max|d| <= 1e-2 max|Y_ref| against oracle.matmul_nbits, over whole and partial
tiles, K tails inside a block and inside a step, odd K-step counts, block
sizes 16 to 128, every zero-point kind and M from 1.
"""
import numpy as np
import pytest

from oracle import oracle as O
from oracle import prepack as PK

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).cuda()


def host(t):
    return t.detach().cpu().numpy()


def ops():
    from xrgpu_amd import ops as _ops
    return _ops


def weights(rng, K, N, bs, zp, bias, dt=np.float16):
    kb = O.k_blocks(K, bs)
    B = rng.integers(0, 256, size=(N, kb, bs // 2), dtype=np.uint8)
    S = rng.uniform(0.001, 0.02, (N, kb)).astype(dt)
    Z = None
    if zp == "packed":
        Z = rng.integers(0, 256, size=(N, O.packed_zp_bytes(kb, 4)), dtype=np.uint8)
    elif zp == "float_int":
        Z = rng.integers(0, 16, size=(N, kb)).astype(dt)
    elif zp == "float":
        Z = rng.uniform(0, 15, (N, kb)).astype(dt)
    b = (rng.standard_normal(N) * 0.1).astype(dt) if bias else None
    return B, S, Z, b


@pytest.mark.parametrize("N,K,bs", [(37, 96, 32), (5, 20, 16), (64, 4096, 128), (1000, 1024, 64), (33, 200, 32)])
def test_prepack_bit_exact(gpu, N, K, bs):
    rng = np.random.default_rng(N + K + bs)
    B = rng.integers(0, 256, size=(N, O.k_blocks(K, bs), bs // 2), dtype=np.uint8)
    got = host(ops().prepack_weights(dev(B), K=K, block_size=bs))
    assert np.array_equal(got, PK.prepack_q4(B, K, bs))


CASES = [
    # M, K, N, bs, zp, bias
    (256, 4096, 512, 128, "packed", True),   # whole tiles, 64 K steps
    (300, 576, 300, 32, None, False),        # 9 K steps (odd), partial tiles both ways
    (513, 256, 257, 16, "packed", False),    # bs = 16: two blocks per chunk
    (130, 200, 33, 32, "packed", True),      # K = 200: 7 blocks, the last K step half empty
    (160, 1024, 96, 64, "float_int", True),
    (140, 512, 72, 128, "float", False),     # float zero points of any value
    (1, 256, 64, 32, None, True),            # one row
    (17, 96, 20, 32, "packed", False),       # K = 96: a K step and a half
    (512, 128, 33768, 128, None, True),      # two row tiles of wide + narrow tiles
]


@pytest.mark.parametrize("M,K,N,bs,zp,bias", CASES)
def test_prepacked_gemm_parity(gpu, M, K, N, bs, zp, bias):
    rng = np.random.default_rng(M * 13 + K + N + bs)
    A = rng.standard_normal((M, K)).astype(np.float16)
    B, S, Z, b = weights(rng, K, N, bs, zp, bias)
    o = ops()
    packed = o.prepack_weights(dev(B), K=K, block_size=bs)
    Y = host(o.matmul_nbits_prepacked(dev(A), packed, dev(S), dev(Z), dev(b), K=K, N=N, block_size=bs))
    ref = O.matmul_nbits(A, B, S, Z, b, K=K, N=N, block_size=bs)
    ok, err, lim = O.tolerance_ok(Y, ref, np.float16)
    assert ok, f"max|d|={err} > {lim}"


def test_prepacked_matches_the_unpacked_gemm(gpu):
    """Same weights, both layouts: the outputs agree to float32 summation order
    (the K order inside each 16-wide MFMA slice differs)."""
    rng = np.random.default_rng(9)
    M, K, N, bs = 512, 2048, 1024, 64
    A = rng.standard_normal((M, K)).astype(np.float16)
    B, S, Z, b = weights(rng, K, N, bs, "packed", True)
    o = ops()
    y1 = host(o.matmul_nbits(dev(A), dev(B), dev(S), dev(Z), dev(b), K=K, N=N, block_size=bs)).astype(np.float32)
    y2 = host(o.matmul_nbits_prepacked(dev(A), o.prepack_weights(dev(B), K=K, block_size=bs), dev(S), dev(Z), dev(b),
                                       K=K, N=N, block_size=bs)).astype(np.float32)
    assert np.max(np.abs(y1 - y2)) <= 2e-3 * np.max(np.abs(y1))


def test_prepacked_rejects_other_geometries(gpu):
    o = ops()
    rng = np.random.default_rng(1)
    A = torch.zeros((4, 64), dtype=torch.float32, device="cuda")
    B, S, _, _ = weights(rng, 64, 8, 32, None, False, np.float32)
    packed = o.prepack_weights(dev(B), K=64, block_size=32)
    from xrgpu_amd import _native as nat
    with pytest.raises(nat.XrmmInvalid, match="prepacked weights run float16"):
        o.matmul_nbits_prepacked(A, packed, dev(S), K=64, N=8, block_size=32)
