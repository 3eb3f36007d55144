"""GPU: the allocation-free int8-activation entry point
(xrmm_matmul_nbits_int8a_noalloc, static device scratch) against the
workspace entry point it varies (xrmm_matmul_nbits_int8a), through the C ABI.

Both run the same kernels on the same inputs, so the outputs must be
bit-identical. Two calls in a row, the second with a smaller input, check that
the shared scratch carries nothing from one call into the next; inputs past the
2 MiB scratch are rejected before any device work.
"""
import numpy as np
import pytest

from xrgpu_amd import _native as nat

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def ops():
    from xrgpu_amd import ops as _ops
    return _ops


def case(rng, M, K, N, bs, dtype, zp):
    kb = K // bs
    A = torch.from_numpy(rng.standard_normal((M, K)).astype(dtype)).cuda()
    B = torch.from_numpy(rng.integers(0, 256, (N, kb, bs // 2), dtype=np.uint8)).cuda()
    S = torch.from_numpy(rng.uniform(0.001, 0.02, (N, kb)).astype(dtype)).cuda()
    Z = torch.from_numpy(rng.integers(0, 256, (N, (kb + 1) // 2), dtype=np.uint8)).cuda() if zp else None
    bias = torch.from_numpy((rng.standard_normal(N) * 0.1).astype(dtype)).cuda()
    return A, B, S, Z, bias


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_noalloc_matches_workspace_entry_two_calls(gpu, dtype):
    rng = np.random.default_rng(41)
    o = ops()
    for M, K, N, bs, zp in ((16, 4096, 1000, 32, True), (3, 1024, 333, 64, False)):
        A, B, S, Z, bias = case(rng, M, K, N, bs, dtype, zp)
        want = o.matmul_nbits_int8a(A, B, S, Z, bias, K=K, N=N, block_size=bs)
        got = o.matmul_nbits_int8a_noalloc(A, B, S, Z, bias, K=K, N=N, block_size=bs)
        torch.cuda.synchronize()
        assert got.shape == (M, N) and got.dtype == want.dtype
        assert torch.equal(got, want), (M, K, N)


def test_noalloc_largest_and_rejected_sizes(gpu):
    rng = np.random.default_rng(42)
    o = ops()
    # 64 rows at K = 16384: 1 MiB of codes + 32 KiB of scales, inside the scratch
    A, B, S, Z, bias = case(rng, 64, 16384, 40, 128, np.float16, True)
    want = o.matmul_nbits_int8a(A, B, S, Z, bias, K=16384, N=40, block_size=128)
    got = o.matmul_nbits_int8a_noalloc(A, B, S, Z, bias, K=16384, N=40, block_size=128)
    assert torch.equal(got, want)
    # 128 rows at K = 16384 need 2 MiB + 64 KiB: rejected, the output untouched
    A2 = torch.zeros((128, 16384), dtype=torch.float16, device="cuda")
    out = torch.full((128, 40), 7.0, dtype=torch.float16, device="cuda")
    with pytest.raises(nat.XrmmInvalid, match="scratch"):
        o.matmul_nbits_int8a_noalloc(A2, B, S, Z, bias, K=16384, N=40, block_size=128, out=out)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
