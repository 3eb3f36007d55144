"""GPU: MatMulNBitsQkv / MatMulNBitsMlp prefill (more than 16 rows) through
the normalisation prologue and the 256 x 256 pipeline, against the oracle.

The prologue writes x = RMSNorm(A + skip) * gamma (or A + skip) once per row
as binary16, rounded after the normalisation (packedInput,
complex_kernel.glsl:81); the GEMM reads x. Covered: the big pipeline's Qkv
grid (three projections on one grid, partial column tiles in each) and Mlp
tiles (gate and up interleaved, every activation, biases, residual), the
128 x 128 fused GEMM on the prologue's output, rows whose un-normalised
(A + skip) * gamma leaves the binary16 range, the workspace-free entry
points, and HIP graph capture. Bars: max|d| <= 1e-2 max|Y_ref| (float16);
the residual A + skip bit-exact."""
import ctypes
import os

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).cuda()


def host(t):
    return None if t is None else t.detach().cpu().numpy()


def ops():
    from xrgpu_amd import ops as _ops
    return _ops


def weights(rng, K, N, bs, zp, bias=False):
    kb = O.k_blocks(K, bs)
    B = rng.integers(0, 256, size=(N, kb, bs // 2), dtype=np.uint8)
    S = rng.uniform(0.001, 0.02, (N, kb)).astype(np.float16)
    Z = None
    if zp == "packed":
        Z = rng.integers(0, 256, size=(N, O.packed_zp_bytes(kb, 4)), dtype=np.uint8)
    elif zp == "float":
        Z = rng.uniform(0, 15, (N, kb)).astype(np.float16)
    b = (rng.standard_normal(N) * 0.1).astype(np.float16) if bias else None
    return B, S, Z, b


def parity(got, ref, what=""):
    ok, err, lim = O.tolerance_ok(host(got) if torch.is_tensor(got) else got, ref, np.float16)
    assert ok, f"{what}: max|d|={err} > {lim}"


@pytest.fixture
def big_threshold():
    """Lets small shapes take the 256 x 256 pipeline (the tile-count
    threshold of the dispatcher, read on every call, set to 0)."""
    old = os.environ.get("XRMM_GEMM_BIG_MIN_TILES")
    os.environ["XRMM_GEMM_BIG_MIN_TILES"] = "0"
    yield
    if old is None:
        del os.environ["XRMM_GEMM_BIG_MIN_TILES"]
    else:
        os.environ["XRMM_GEMM_BIG_MIN_TILES"] = old


def activations(rng, M, K, skip, loud):
    """A and skip ~ N(0, 1), or (loud) binary16 values near the top of the
    range whose sum A + skip reaches 1.2e5 (past 65504) in most elements."""
    if not loud:
        A = rng.standard_normal((M, K)).astype(np.float16)
        return A, (rng.standard_normal((M, K)).astype(np.float16) if skip else None)
    sign = np.where(rng.random((M, K)) < 0.5, -1.0, 1.0)
    A = (sign * rng.uniform(30000, 60000, (M, K))).astype(np.float16)
    return A, (sign * rng.uniform(30000, 60000, (M, K))).astype(np.float16)


def run_qkv(rng, M, K, Nq, Nkv, bs, zp, skip, loud=False, rows=None):
    A, sk = activations(rng, M, K, skip, loud)
    g = rng.uniform(0.5, 1.5, K).astype(np.float16)
    parts = [weights(rng, K, n, bs, zp)[:3] for n in (Nq, Nkv, Nkv)]
    Q, Kk, V, R = ops().matmul_nbits_qkv(dev(A), *[dev(x) for p in parts for x in p[:2]], norm_scale=dev(g),
                                         skip=dev(sk), block_size=bs, q_zero_points=dev(parts[0][2]),
                                         k_zero_points=dev(parts[1][2]), v_zero_points=dev(parts[2][2]))
    sel = slice(None) if rows is None else rows
    ref = O.matmul_nbits_qkv(A[sel], parts[0][0], parts[0][1], parts[1][0], parts[1][1], parts[2][0], parts[2][1],
                             K=K, Nq=Nq, Nkv=Nkv, norm_scale=g, skip=None if sk is None else sk[sel], block_size=bs,
                             q_zero_points=parts[0][2], k_zero_points=parts[1][2], v_zero_points=parts[2][2])
    for got, exp, nm in zip((Q, Kk, V), ref[:3], "qkv"):
        parity(host(got)[sel], exp, nm)
    assert np.array_equal(host(R)[sel].view(np.uint16), ref[3].view(np.uint16))


QKV_BIG = [
    # M, K, Nq, Nkv, bs, zp, skip
    (256, 512, 1024, 256, 64, "packed", True),    # whole tiles, packed zero points
    (384, 320, 1000, 200, 32, None, False),       # partial row tile, partial column tiles in all three
    (128, 256, 512, 136, 16, "float", True),      # block_size 16, float zero points
    (300, 1024, 520, 24, 128, "packed", False),   # a projection narrower than a tile
]


@pytest.mark.parametrize("M,K,Nq,Nkv,bs,zp,skip", QKV_BIG)
def test_qkv_big_pipeline(gpu, big_threshold, M, K, Nq, Nkv, bs, zp, skip):
    kind = None if zp is None else zp
    assert ops().select_kernel("MatMulNBitsQkv", M, K, Nq, 4, bs, torch.float16, kind) == "gemm_q4_big_fused"
    run_qkv(np.random.default_rng(M + K + Nq + bs), M, K, Nq, Nkv, bs, zp, skip)


def test_qkv_prefill_full_size_row_sample(gpu):
    """The GQA prefill layout at 2048 rows (192 tiles, the default threshold),
    checked on a seeded sample of rows (rows are independent)."""
    M, K, Nq, Nkv, bs = 2048, 4096, 4096, 1024, 64
    assert ops().select_kernel("MatMulNBitsQkv", M, K, Nq, 4, bs, torch.float16, "packed") == "gemm_q4_big_fused"
    rng = np.random.default_rng(2048)
    rows = np.sort(rng.choice(M, 96, replace=False))
    run_qkv(rng, M, K, Nq, Nkv, bs, "packed", True, rows=rows)


def run_mlp(rng, M, K, N, bs, zp, skip, norm, biases, act, res, loud=False, rows=None):
    A, sk = activations(rng, M, K, skip, loud)
    g = rng.uniform(0.5, 1.5, K).astype(np.float16) if norm else None
    gB, gS, gZ, gb = weights(rng, K, N, bs, zp, biases)
    uB, uS, uZ, ub = weights(rng, K, N, bs, zp, biases)
    Y, R = ops().matmul_nbits_mlp(dev(A), dev(gB), dev(gS), dev(uB), dev(uS), skip=dev(sk), norm_scale=dev(g),
                                  gate_bias=dev(gb), up_bias=dev(ub), block_size=bs, activation=act,
                                  gate_zero_points=dev(gZ), up_zero_points=dev(uZ), want_residual=res)
    sel = slice(None) if rows is None else rows
    ref, r = O.matmul_nbits_mlp(A[sel], gB, gS, uB, uS, K=K, N=N, skip=None if sk is None else sk[sel],
                                norm_scale=g, gate_bias=gb, up_bias=ub, block_size=bs, activation=act,
                                gate_zero_points=gZ, up_zero_points=uZ)
    parity(host(Y)[sel], ref, "mlp")
    if res:
        assert np.array_equal(host(R)[sel].view(np.uint16), r.view(np.uint16))
    return A, sk, g


MLP_BIG = [
    # M, K, N, bs, zp, skip, norm, biases, act, residual
    (256, 512, 1024, 32, None, False, True, False, "silu", False),    # the SwiGLU layout
    (300, 384, 1000, 64, "packed", True, True, True, "gelu", True),   # partial tiles, residual
    (128, 256, 200, 16, "float", True, False, True, "relu", True),    # skip without norm, block_size 16
    (256, 256, 640, 128, None, False, False, False, "none", False),   # no prologue at all
    (200, 256, 136, 32, "packed", False, True, True, "tanh", False),
    (256, 256, 256, 32, None, True, True, False, "sigmoid", True),
    (256, 256, 40000, 32, "packed", True, True, True, "silu", True),  # 313 tiles: wide and narrow (64-output) tiles
]


@pytest.mark.parametrize("M,K,N,bs,zp,skip,norm,biases,act,res", MLP_BIG)
def test_mlp_big_pipeline(gpu, big_threshold, M, K, N, bs, zp, skip, norm, biases, act, res):
    kind = None if zp is None else zp
    assert ops().select_kernel("MatMulNBitsMlp", M, K, N, 4, bs, torch.float16, kind) == "gemm_q4_big_fused"
    run_mlp(np.random.default_rng(M * 3 + K + N), M, K, N, bs, zp, skip, norm, biases, act, res)


def test_mlp_prefill_full_size_row_sample(gpu):
    """The Llama-3-8B SwiGLU prefill layout (M = 2048, K = 4096, N = 14336:
    896 tiles) on a seeded sample of rows."""
    M, K, N, bs = 2048, 4096, 14336, 32
    assert ops().select_kernel("MatMulNBitsMlp", M, K, N, 4, bs, torch.float16, None) == "gemm_q4_big_fused"
    rng = np.random.default_rng(14336)
    rows = np.sort(rng.choice(M, 64, replace=False))
    run_mlp(rng, M, K, N, bs, None, False, True, False, "silu", False, rows=rows)


@pytest.mark.parametrize("op,M", [("qkv", 100), ("qkv", 256), ("mlp", 100), ("mlp", 256)])
def test_unnormalised_rows_beyond_binary16(gpu, op, M):
    """|A + skip| reaches 1.2e5 (past 65504) while the normalised rows stay
    small: the prologue rounds after normalising, so the outputs are finite
    and meet the oracle on the 128 x 128 GEMM (100 rows) and the big pipeline
    (256 rows); the residual A + skip overflows to +-Inf exactly as the
    oracle's binary16 rounding of it does."""
    rng = np.random.default_rng(65504 + M)
    os.environ["XRMM_GEMM_BIG_MIN_TILES"] = "0" if M >= 128 else "128"
    try:
        if op == "qkv":
            K, Nq, Nkv, bs = 256, 256, 64, 32
            want = "gemm_q4_big_fused" if M >= 128 else "gemm_q4_fused"
            assert ops().select_kernel("MatMulNBitsQkv", M, K, Nq, 4, bs, torch.float16, None) == want
            run_qkv(rng, M, K, Nq, Nkv, bs, None, True, loud=True)
        else:
            K, N, bs = 256, 256, 32
            want = "gemm_q4_big_fused" if M >= 128 else "gemm_q4_fused"
            assert ops().select_kernel("MatMulNBitsMlp", M, K, N, 4, bs, torch.float16, None) == want
            run_mlp(rng, M, K, N, bs, None, True, True, False, "silu", True, loud=True)
    finally:
        del os.environ["XRMM_GEMM_BIG_MIN_TILES"]


def test_workspace_free_entry_points_still_normalise_in_place(gpu):
    """xrmm_matmul_nbits_qkv / _mlp without a workspace run the 128 x 128
    GEMM, which normalises inside its K loop, for prefill geometries too."""
    from xrgpu_amd import _native as nat
    lib = nat.lib()
    rng = np.random.default_rng(77)
    M, K, N, bs = 256, 512, 1024, 32
    A = rng.standard_normal((M, K)).astype(np.float16)
    g = rng.uniform(0.5, 1.5, K).astype(np.float16)
    gB, gS, _, _ = weights(rng, K, N, bs, None)
    uB, uS, _, _ = weights(rng, K, N, bs, None)
    d = [dev(x) for x in (A, g, gB, gS, uB, uS)]
    Y = torch.empty((M, N), dtype=torch.float16, device="cuda")
    p = lambda t: None if t is None else t.data_ptr()
    nat.check(lib.xrmm_matmul_nbits_mlp(p(d[0]), None, p(d[1]), p(d[2]), p(d[3]), None, None, p(d[4]), p(d[5]),
                                        None, None, nat.UNSPECIFIED, p(Y), None, M, K, N, 4, bs, 1e-5,
                                        nat.ACT["silu"], nat.F16, None))
    torch.cuda.synchronize()
    ref, _ = O.matmul_nbits_mlp(A, gB, gS, uB, uS, K=K, N=N, norm_scale=g, block_size=bs)
    parity(host(Y), ref, "mlp without workspace")
    assert lib.xrmm_matmul_nbits_fused_workspace_bytes(2, M, K, N, 0, 4, bs, nat.F16, 0, 1) == M * K * 2


def test_fused_prefill_under_graph_capture(gpu, big_threshold):
    """The prologue + big-pipeline Mlp and Qkv captured into one graph (the
    workspaces come from the graph's pool), replayed three times with eager
    calls and synchronisations between; every replay meets the oracle."""
    rng = np.random.default_rng(91)
    M, K, N, bs = 256, 512, 2048, 32
    A = rng.standard_normal((M, K)).astype(np.float16)
    g = rng.uniform(0.5, 1.5, K).astype(np.float16)
    gB, gS, _, _ = weights(rng, K, N, bs, None)
    uB, uS, _, _ = weights(rng, K, N, bs, None)
    qkv = [weights(rng, K, n, bs, None)[:2] for n in (2048, 512, 512)]
    d = dict(A=dev(A), g=dev(g), gB=dev(gB), gS=dev(gS), uB=dev(uB), uS=dev(uS))
    dq = [[dev(x) for x in p] for p in qkv]
    o = ops()
    assert o.select_kernel("MatMulNBitsMlp", M, K, N, 4, bs, torch.float16, None) == "gemm_q4_big_fused"
    assert o.select_kernel("MatMulNBitsQkv", M, K, 2048, 4, bs, torch.float16, None) == "gemm_q4_big_fused"

    def step():
        y, _ = o.matmul_nbits_mlp(d["A"], d["gB"], d["gS"], d["uB"], d["uS"], norm_scale=d["g"], block_size=bs)
        q = o.matmul_nbits_qkv(d["A"], *[x for p in dq for x in p], norm_scale=d["g"], block_size=bs,
                               want_residual=False)
        return y, q[0]

    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y_g, q_g = step()
    ref_y, _ = O.matmul_nbits_mlp(A, gB, gS, uB, uS, K=K, N=N, norm_scale=g, block_size=bs)
    ref_q = O.matmul_nbits_qkv(A, *[x for p in qkv for x in p], K=K, Nq=2048, Nkv=512, norm_scale=g,
                               block_size=bs)[0]
    for rep in range(3):
        y_g.zero_()
        q_g.zero_()
        graph.replay()
        torch.cuda.synchronize()
        parity(host(y_g), ref_y, f"mlp replay {rep}")
        parity(host(q_g), ref_q, f"qkv replay {rep}")
        y_e, q_e = step()  # eager work between replays
        torch.cuda.synchronize()
        parity(host(y_e), ref_y, "mlp eager")
