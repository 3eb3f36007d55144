"""MatMulNBits split over K across workgroups (xrmm_matmul_nbits_ws), against
the oracle: float32 partial tiles in a workspace, added by each tile's last
split in split order. Bars: the float16 bar max|d| <= 1e-2 max|Y_ref|;
repeated calls on one workspace give bitwise-identical outputs (the split
order is fixed and the workspace is left zero-filled); the workspace-free
entry point agrees within the bar."""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).cuda()


def host(t):
    return t.detach().cpu().numpy()


def ops():
    from xrgpu_amd import ops as _ops
    return _ops


def case(rng, M, K, N, bs, zp, bias):
    kb = O.k_blocks(K, bs)
    A = rng.standard_normal((M, K)).astype(np.float16)
    B = rng.integers(0, 256, size=(N, kb, bs // 2), dtype=np.uint8)
    S = rng.uniform(0.001, 0.02, (N, kb)).astype(np.float16)
    Z = None
    if zp == "packed":
        Z = rng.integers(0, 256, size=(N, O.packed_zp_bytes(kb, 4)), dtype=np.uint8)
    elif zp == "float":
        Z = rng.uniform(0, 15, (N, kb)).astype(np.float16)
    b = (rng.standard_normal(N) * 0.1).astype(np.float16) if bias else None
    return A, B, S, Z, b


CASES = [
    # M, K, N, bs, zp, bias: the down projection (32 tiles, 8 splits), rows
    # past the split-K GEMV, a partial last split, few columns, float zero points
    (128, 14336, 4096, 128, "packed", True),
    (64, 14336, 4096, 64, None, False),
    (100, 4096, 14336, 32, "packed", True),
    (17, 8192, 512, 32, None, True),
    (200, 1056, 300, 32, "float", False),     # 17 K steps: the last split is shorter
    (33, 2080, 130, 16, "packed", True),      # bs = 16
]


@pytest.mark.parametrize("M,K,N,bs,zp,bias", CASES)
def test_splitk_gemm_parity(gpu, M, K, N, bs, zp, bias):
    from xrgpu_amd import _native as nat
    assert nat.lib().xrmm_matmul_nbits_workspace_bytes(M, K, N, 4, bs, nat.F16) > 0
    rng = np.random.default_rng(M * 3 + K + N + bs)
    A, B, S, Z, b = case(rng, M, K, N, bs, zp, bias)
    Y = host(ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), dev(b), K=K, N=N, block_size=bs))
    ref = O.matmul_nbits(A, B, S, Z, b, K=K, N=N, block_size=bs)
    ok, err, lim = O.tolerance_ok(Y, ref, np.float16)
    assert ok, f"max|d|={err} > {lim}"


def test_splitk_repeat_is_bitwise_and_workspace_stays_zero(gpu):
    from xrgpu_amd import _native as nat
    rng = np.random.default_rng(4)
    M, K, N, bs = 96, 14336, 4096, 128
    A, B, S, Z, b = case(rng, M, K, N, bs, "packed", True)
    need = nat.lib().xrmm_matmul_nbits_workspace_bytes(M, K, N, 4, bs, nat.F16)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    tA, tB, tS, tZ, tb = dev(A), dev(B), dev(S), dev(Z), dev(b)
    outs = []
    for _ in range(3):
        Y = torch.empty((M, N), dtype=torch.float16, device="cuda")
        nat.check(nat.lib().xrmm_matmul_nbits_ws(tA.data_ptr(), tB.data_ptr(), tS.data_ptr(), tZ.data_ptr(), nat.U8,
                                                 tb.data_ptr(), Y.data_ptr(), M, K, N, 4, bs, nat.F16, ws.data_ptr(),
                                                 need, None))
        torch.cuda.synchronize()
        outs.append(host(Y))
        assert not ws[:4096].any().item()  # every tile's counter back at zero
    assert np.array_equal(outs[0].view(np.uint16), outs[1].view(np.uint16))
    assert np.array_equal(outs[0].view(np.uint16), outs[2].view(np.uint16))
    # the workspace-free entry point (one split per tile) agrees within the bar
    Y1 = torch.empty((M, N), dtype=torch.float16, device="cuda")
    nat.check(nat.lib().xrmm_matmul_nbits(tA.data_ptr(), tB.data_ptr(), tS.data_ptr(), tZ.data_ptr(), nat.U8,
                                          tb.data_ptr(), Y1.data_ptr(), M, K, N, 4, bs, nat.F16, None))
    torch.cuda.synchronize()
    ok, err, lim = O.tolerance_ok(host(Y1), outs[0].astype(np.float32), np.float16)
    assert ok, (err, lim)


def test_splitk_workspace_shared_between_shapes(gpu):
    """One workspace, calls of different shapes in turn (different tile counts
    and splits): the counters sit in a fixed block, so a larger geometry never
    reads a smaller one's partial tiles as counters."""
    from xrgpu_amd import _native as nat
    shapes = [(17, 8192, 512, 32), (100, 4096, 14336, 32), (64, 14336, 4096, 128), (100, 4096, 14336, 32)]
    need = max(nat.lib().xrmm_matmul_nbits_workspace_bytes(M, K, N, 4, bs, nat.F16) for M, K, N, bs in shapes)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    for M, K, N, bs in shapes:
        rng = np.random.default_rng(M + K + N)
        A, B, S, Z, b = case(rng, M, K, N, bs, "packed", True)
        tA, tB, tS, tZ, tb = dev(A), dev(B), dev(S), dev(Z), dev(b)
        Y = torch.empty((M, N), dtype=torch.float16, device="cuda")
        nat.check(nat.lib().xrmm_matmul_nbits_ws(tA.data_ptr(), tB.data_ptr(), tS.data_ptr(), tZ.data_ptr(), nat.U8,
                                                 tb.data_ptr(), Y.data_ptr(), M, K, N, 4, bs, nat.F16, ws.data_ptr(),
                                                 need, None))
        ok, err, lim = O.tolerance_ok(host(Y), O.matmul_nbits(A, B, S, Z, b, K=K, N=N, block_size=bs), np.float16)
        assert ok, ((M, K, N), err, lim)


def test_splitk_rejects_a_short_workspace(gpu):
    from xrgpu_amd import _native as nat
    M, K, N, bs = 64, 14336, 4096, 128
    need = nat.lib().xrmm_matmul_nbits_workspace_bytes(M, K, N, 4, bs, nat.F16)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    x = torch.zeros(16, dtype=torch.float16, device="cuda")
    rc = nat.lib().xrmm_matmul_nbits_ws(x.data_ptr(), x.data_ptr(), x.data_ptr(), None, nat.UNSPECIFIED, None,
                                        x.data_ptr(), M, K, N, 4, bs, nat.F16, ws.data_ptr(), need - 1, None)
    assert rc == nat.XRMM_EINVAL and "workspace" in nat.last_error()


def _check(y, A, B, S, Z, b, K, N, bs):
    ref = O.matmul_nbits(A, B, S, Z, b, K=K, N=N, block_size=bs)
    ok, err, lim = O.tolerance_ok(host(y), ref, np.float16)
    assert ok, (err, lim)


@pytest.mark.parametrize("caller_workspace", [False, True])
def test_splitk_geometries_under_graph_capture(gpu, caller_workspace):
    """Two split-K geometries captured into two graphs on torch's shared
    capture stream, the smaller one replayed first, each replayed several
    times with eager split-K calls and synchronisations in between; every
    replay meets the oracle. Without a caller workspace the captured calls
    run unsplit (nothing captured depends on the front end's own
    workspaces); with one workspace per graph, allocated and zero-filled
    outside capture, they run split."""
    rng = np.random.default_rng(61)
    shapes = [(40, 8192, 512, 64), (17, 8192, 512, 32)]
    cases = [case(rng, M, K, N, bs, "packed", True) for M, K, N, bs in shapes]
    dv = [[dev(x) for x in c] for c in cases]
    outs = [torch.empty((M, N), dtype=torch.float16, device="cuda") for M, K, N, bs in shapes]
    ws = [torch.zeros(ops().matmul_nbits_workspace_bytes(M, K, N, 4, bs), dtype=torch.uint8, device="cuda")
          if caller_workspace else None for M, K, N, bs in shapes]
    assert all(ops().matmul_nbits_workspace_bytes(M, K, N, 4, bs) > 0 for M, K, N, bs in shapes)

    def call(i):
        A, B, S, Z, b = dv[i]
        M, K, N, bs = shapes[i]
        ops().matmul_nbits(A, B, S, Z, b, block_size=bs, out=outs[i], workspace=ws[i])

    for i in range(2):  # warm-up outside capture
        call(i)
    torch.cuda.synchronize()
    graphs = []
    for i in range(2):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            call(i)
        graphs.append(g)
    torch.cuda.synchronize()
    for rep in range(3):
        for i in (1, 0):  # the smaller graph first
            outs[i].zero_()
            graphs[i].replay()
            torch.cuda.synchronize()
            _check(outs[i], *cases[i], shapes[i][1], shapes[i][2], shapes[i][3])
            # eager split-K work on the default stream between replays
            A, B, S, Z, b = dv[1 - i]
            M, K, N, bs = shapes[1 - i]
            y = ops().matmul_nbits(A, B, S, Z, b, block_size=bs)
            torch.cuda.synchronize()
            _check(y, *cases[1 - i], K, N, bs)
