"""Size limits of MatMulNBits on the GPU.

The fast kernels address weights through 32-bit buffer ranges and take
geometries whose code bytes stay under 2^30; larger ones go to the generic
kernel (64-bit indexing). These cases sit on both sides of that line and
past 2^31 bytes, plus the prefill GEMM on a grid of 2048 tiles (256-wide
tiles, then 192-wide ones). Weights are generated on the device; columns
are independent, so the oracle checks a seeded sample of them (always
including the first and the last two).
"""
import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def ops():
    from xrgpu_amd import ops as _ops
    return _ops


def host(t):
    return t.detach().cpu().numpy()


LIMIT_CASES = [
    # M, N, kernel: K = 4096, block 32, 4-bit, packed zero points (2 KB of codes per column)
    (1, 524287, "gemv_q4_dot"),     # codes 1 GiB - 2 KB: the largest fast geometry
    (4, 524287, "gemv_q4_splitk"),
    (40, 524287, "gemv_q4_splitk"),  # three row chunks at the largest geometry
    (1, 524288, "generic"),         # codes exactly 1 GiB
    (2, 1048577, "generic"),        # codes 2 GiB + 2 KB: offsets past 2^31
    (256, 524287, "gemm_q4_big"),   # 2048 tiles of 256 x 256, then 256 x 192
]


@pytest.mark.parametrize("M,N,kernel", LIMIT_CASES)
def test_size_limits(gpu, M, N, kernel):
    K, bs = 4096, 32
    kb = K // bs
    assert ops().select_kernel("MatMulNBits", M, K, N, 4, bs, torch.float16, "packed") == kernel
    g = torch.Generator(device="cuda").manual_seed(M * 1000003 + N)
    B = torch.randint(0, 256, (N, kb, 16), dtype=torch.uint8, device="cuda", generator=g)
    S = (torch.rand((N, kb), device="cuda", generator=g) * 0.02 + 0.001).half()
    Z = torch.randint(0, 256, (N, kb // 2), dtype=torch.uint8, device="cuda", generator=g)
    A = torch.randn((M, K), device="cuda", generator=g).half()
    Y = ops().matmul_nbits(A, B, S, Z, None, K=K, N=N, block_size=bs)
    rng = np.random.default_rng(N)
    cols = np.unique(np.concatenate([[0, N - 2, N - 1], rng.choice(N, 160, replace=False)]))
    ci = torch.from_numpy(cols).cuda()
    ref = O.matmul_nbits(host(A), host(B[ci]), host(S[ci]), host(Z[ci]), None, K=K, N=len(cols), block_size=bs)
    ok, err, lim = O.tolerance_ok(host(Y[:, ci]), ref, np.float16)
    assert ok, f"max|d|={err} > {lim}"
