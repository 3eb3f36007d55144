"""GPU: non-finite activations and large scales, every kernel family, against
the oracle's policy.

The reference accumulates ``sum += a * W`` serially in float32
(complex_kernel.glsl:83) with ``W = (code - z) * scale`` (:80): an activation
of +-Inf gives +-Inf (NaN where W is 0, or where +Inf and -Inf terms meet), a
NaN activation gives NaN. With RMS normalisation (Qkv, Mlp with normScale) an
infinite row has sum(r^2) = Inf, so inversesqrt gives 0 and x = Inf * 0 = NaN
for the whole row (:81). The oracle's non-finite pattern is pinned to the
serial float32 restatement (tests/test_oracle.py); here every kernel family
must reproduce it exactly (``tolerance_ok``: same +-Inf, NaN where NaN) and the
finite rows within the usual bar.

Large scales: binary16 kernels that stage dequantised weights in binary16
would saturate |(code - z) * scale| > 65504 to +-Inf, where the reference's
float32 weight is finite. Within that range every kernel is exact; beyond it
the request lifecycle (which holds the scales on the host) routes the call to
kernels that keep weights in float32.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.test_oracle import nonfinite_activations
from xrgpu_amd import operator as op

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).cuda()


def host(t):
    return None if t is None else t.detach().cpu().numpy()


def ops():
    from xrgpu_amd import ops as _ops
    return _ops


def weights(rng, K, N, bs, dtype, zp, scale_lo=0.01, scale_hi=0.2):
    kb = O.k_blocks(K, bs)
    B = rng.integers(0, 256, (N, kb, bs // 2), dtype=np.uint8)
    S = rng.uniform(scale_lo, scale_hi, (N, kb)).astype(dtype)
    Z = None
    if zp == "packed":
        Z = rng.integers(0, 256, (N, O.packed_zp_bytes(kb, 4)), dtype=np.uint8)
    elif zp == "float":
        Z = rng.integers(0, 16, (N, kb)).astype(dtype)
    return B, S, Z


def zkind(zp):
    return None if zp is None else ("packed" if zp == "packed" else "float")


MNB_CASES = [
    # M, K, N, bs, dtype, zp, expected kernel family
    (1, 1024, 64, 32, np.float16, None, "gemv_q4_dot"),
    (2, 2048, 96, 64, np.float16, "packed", "gemv_q4_dot"),
    (2, 512, 40, 16, np.float16, "float", "gemv_q4_dot"),
    (5, 2048, 64, 32, np.float16, None, "gemv_q4_splitk"),
    (8, 4096, 40, 64, np.float16, "packed", "gemv_q4_splitk"),
    (5, 512, 48, 16, np.float16, "packed", "gemv_q4_mfma"),
    (48, 512, 128, 32, np.float16, "packed", "gemm_q4_thin"),
    (128, 512, 256, 64, np.float16, "float", "gemm_q4_mfma"),
    (2048, 256, 4096, 64, np.float16, "packed", "gemm_q4_big"),
    (5, 96, 40, 32, np.float32, "packed", "gemv_q4_f32"),   # float32 rows in chunks of four
    (5, 98, 40, 32, np.float32, "packed", "generic"),       # K % 4 != 0
    (4, 96, 40, 32, np.float32, "packed", "gemv_q4_f32"),
    (3, 2048, 33, 64, np.float32, "float", "gemv_q4_f32"),
    (1, 4096, 64, 16, np.float32, None, "gemv_q4_f32"),
    (4, 100, 17, 32, np.float16, None, "generic"),   # K % 8 != 0
    (48, 512, 128, 32, np.float32, "packed", "gemm_f32_mfma"),  # float32 prefill rows
    (40, 1024, 96, 64, np.float32, "float", "gemm_f32_mfma"),   # float zero points: rows recomputed
]


@pytest.mark.parametrize("M,K,N,bs,dtype,zp,family", MNB_CASES)
def test_matmul_nbits_nonfinite_activations(gpu, M, K, N, bs, dtype, zp, family):
    rng = np.random.default_rng(M * 7 + K + N)
    assert ops().select_kernel("MatMulNBits", M, K, N, 4, bs, torch.float16 if dtype == np.float16 else torch.float32,
                               zkind(zp)) == family
    A = nonfinite_activations(rng, M, K, dtype)
    B, S, Z = weights(rng, K, N, bs, dtype, zp)
    bias = (rng.standard_normal(N) * 0.1).astype(dtype)
    Y = host(ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), dev(bias), K=K, N=N, block_size=bs))
    ref = O.matmul_nbits(A, B, S, Z, bias, K=K, N=N, block_size=bs)
    ok, err, lim = O.tolerance_ok(Y, ref, dtype)
    assert ok, (family, err, lim, np.argwhere(~(np.isfinite(Y) == np.isfinite(ref)))[:5])
    assert not np.all(np.isfinite(ref[0]))  # the case really carries non-finite outputs


def test_dot_gemv_finite_workgroups_unaffected(gpu):
    """One infinite activation routes the workgroups of that launch to the
    per-element form; a second call with finite activations on the same
    weights must give the usual fast-path result (no state carries over)."""
    rng = np.random.default_rng(5)
    K, N, bs = 4096, 1000, 32
    B, S, _ = weights(rng, K, N, bs, np.float16, None)
    A = rng.standard_normal((1, K)).astype(np.float16)
    Ai = A.copy()
    Ai[0, 17] = np.inf
    o = ops()
    y1 = host(o.matmul_nbits(dev(Ai), dev(B), dev(S), K=K, N=N, block_size=bs))
    y2 = host(o.matmul_nbits(dev(A), dev(B), dev(S), K=K, N=N, block_size=bs))
    assert O.tolerance_ok(y1, O.matmul_nbits(Ai, B, S, K=K, N=N, block_size=bs), np.float16)[0]
    assert O.tolerance_ok(y2, O.matmul_nbits(A, B, S, K=K, N=N, block_size=bs), np.float16)[0]


QKV_CASES = [
    # M, K, Nq, Nkv, bs, dtype, skip_nonfinite, expected family
    (4, 2048, 64, 32, 32, np.float16, False, "gemv_q4_mq"),
    (2, 1024, 40, 24, 64, np.float16, True, "gemv_q4_mq"),
    (3, 1024, 40, 24, 16, np.float16, True, "gemv_q4_dot"),
    (8, 2048, 64, 32, 32, np.float16, False, "gemv_q4_splitk"),
    (32, 1024, 40, 24, 32, np.float16, False, "gemm_q4_fused"),
    (20, 512, 130, 3, 16, np.float16, True, "gemm_q4_fused"),
    (5, 96, 16, 8, 32, np.float32, True, "f32_proj"),
    (40, 1024, 64, 32, 64, np.float32, True, "f32_proj"),   # more than 16 rows: the MFMA GEMM per projection
]


@pytest.mark.parametrize("M,K,Nq,Nkv,bs,dtype,skip_nf,family", QKV_CASES)
def test_qkv_nonfinite_rows(gpu, M, K, Nq, Nkv, bs, dtype, skip_nf, family):
    """Infinite or NaN inputs make the whole normalised row NaN
    (inversesqrt(Inf) = 0, Inf * 0 = NaN); the other rows stay finite."""
    rng = np.random.default_rng(M * 11 + K + Nq)
    t = torch.float16 if dtype == np.float16 else torch.float32
    assert ops().select_kernel("MatMulNBitsQkv", M, K, Nq, 4, bs, t) == family
    sk = rng.standard_normal((M, K)).astype(dtype)
    if skip_nf:
        A = rng.standard_normal((M, K)).astype(dtype)
        sk[0, 3], sk[1, 9] = np.inf, np.nan
    else:
        A = nonfinite_activations(rng, M, K, dtype)
    g = rng.uniform(0.5, 1.5, K).astype(dtype)
    parts = [weights(rng, K, n, bs, dtype, None)[:2] for n in (Nq, Nkv, Nkv)]
    Q, Kk, V, R = ops().matmul_nbits_qkv(dev(A), *[dev(x) for p in parts for x in p], norm_scale=dev(g),
                                         skip=dev(sk), block_size=bs)
    ref = O.matmul_nbits_qkv(A, parts[0][0], parts[0][1], parts[1][0], parts[1][1], parts[2][0], parts[2][1],
                             K=K, Nq=Nq, Nkv=Nkv, norm_scale=g, skip=sk, block_size=bs)
    for got, exp in zip((Q, Kk, V), ref[:3]):
        ok, err, lim = O.tolerance_ok(host(got), exp, dtype)
        assert ok, (family, err, lim)
        assert np.isnan(exp[0]).all() and np.isnan(exp[1]).all()
        assert np.isfinite(exp[4:]).all()
    assert O.tolerance_ok(host(R), ref[3], dtype)[0]


MLP_CASES = [
    # M, K, N, bs, dtype, norm, expected family
    (8, 2048, 64, 32, np.float16, False, "gemv_q4_splitk"),
    (6, 1024, 40, 64, np.float16, True, "gemv_q4_mfma"),
    (24, 2048, 64, 32, np.float16, False, "gemm_q4_thin"),      # 17..64 rows: the thin GEMM
    (70, 1024, 64, 32, np.float16, False, "gemm_q4_fused"),
    (130, 1024, 40, 64, np.float16, True, "gemm_q4_fused"),
    (4, 96, 24, 32, np.float32, False, "f32_proj"),
    (4, 96, 24, 32, np.float32, True, "f32_proj"),
    (48, 1024, 64, 64, np.float32, True, "f32_proj"),
]


@pytest.mark.parametrize("M,K,N,bs,dtype,norm,family", MLP_CASES)
def test_mlp_nonfinite_activations(gpu, M, K, N, bs, dtype, norm, family):
    """silu(+Inf) * u = +-Inf, silu(-Inf) = -Inf * logistic(-Inf) = NaN
    (complex_kernel.glsl:39,41); with normScale infinite rows turn NaN."""
    rng = np.random.default_rng(M * 13 + K + N)
    t = torch.float16 if dtype == np.float16 else torch.float32
    assert ops().select_kernel("MatMulNBitsMlp", M, K, N, 4, bs, t) == family
    A = nonfinite_activations(rng, M, K, dtype)
    g = rng.uniform(0.5, 1.5, K).astype(dtype) if norm else None
    gB, gS, _ = weights(rng, K, N, bs, dtype, None)
    uB, uS, _ = weights(rng, K, N, bs, dtype, None)
    Y, _ = ops().matmul_nbits_mlp(dev(A), dev(gB), dev(gS), dev(uB), dev(uS), norm_scale=dev(g), block_size=bs)
    ref, _ = O.matmul_nbits_mlp(A, gB, gS, uB, uS, K=K, N=N, norm_scale=g, block_size=bs)
    ok, err, lim = O.tolerance_ok(host(Y), ref, dtype)
    assert ok, (family, err, lim)
    assert not np.isfinite(ref[0]).all()


@pytest.mark.parametrize("M,K,N,bs,zp,family", [(1, 1024, 64, 32, None, "gemv_q4_dot"),
                                                 (5, 2048, 64, 32, "packed", "gemv_q4_splitk"),
                                                 (48, 512, 128, 32, "packed", "gemm_q4_thin"),
                                                 (128, 512, 256, 64, "float", "gemm_q4_mfma"),
                                                 (2048, 256, 4096, 64, "packed", "gemm_q4_big")])
def test_large_scales_within_binary16_weight_range(gpu, M, K, N, bs, zp, family):
    """Scales up to 4000 keep every binary16 weight finite (15 * 4000 < 65504;
    the binary16 scale nearest 65504 / 15 is 4368, whose 15-fold is 65520 and
    rounds to +Inf): each kernel family matches the oracle with such scales
    (tiny activations keep Y in range)."""
    rng = np.random.default_rng(M + K + N + 1)
    assert ops().select_kernel("MatMulNBits", M, K, N, 4, bs, torch.float16, zkind(zp)) == family
    A = (rng.standard_normal((M, K)) * 1e-3).astype(np.float16)
    B, S, Z = weights(rng, K, N, bs, np.float16, zp, scale_lo=1000.0, scale_hi=4000.0)
    Y = host(ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), K=K, N=N, block_size=bs))
    ref = O.matmul_nbits(A, B, S, Z, K=K, N=N, block_size=bs)
    ok, err, lim = O.tolerance_ok(Y, ref, np.float16)
    assert ok and np.isfinite(ref).all(), (family, err, lim)


@pytest.mark.parametrize("M,K,N,bs", [(1, 1024, 64, 32), (5, 2048, 64, 32), (48, 512, 128, 32), (300, 1024, 96, 64)])
def test_lifecycle_scales_beyond_binary16_weight_range(gpu, M, K, N, bs):
    """Scales of 30000 with an implicit zero point give float32 weights up to
    240000 (finite in the reference, beyond binary16). The request lifecycle
    checks the scales at prepare and runs kernels that keep weights in
    float32 (the dot GEMV for up to two rows, the float32-arithmetic GEMV up
    to 16, the float32-arithmetic GEMM beyond); the result matches the
    oracle."""
    rng = np.random.default_rng(M + K + N + 2)
    kb = K // bs
    ins = dict(aT=(rng.standard_normal((M, K)) * 1e-4).astype(np.float16),
               bT=rng.integers(0, 256, (N, kb, bs // 2), dtype=np.uint8),
               scalesT=rng.uniform(20000.0, 30000.0, (N, kb)).astype(np.float16))
    req = op.Request("com.microsoft.MatMulNBits", [op.Tensor(k, v) for k, v in ins.items()],
                     attrs={"N": N, "block_size": bs})
    with op.Operator.prepare("", req) as o:
        o.run()
        (y,) = o.read_outputs()
        info = o.info()
    ref = O.matmul_nbits(ins["aT"], ins["bT"], ins["scalesT"], K=K, N=N, block_size=bs)
    assert np.isfinite(ref).all()
    ok, err, lim = O.tolerance_ok(y.data, ref, np.float16)
    assert ok, (info.get("kernel"), err, lim)
    assert info.get("kernel") == ("gemv_q4_dot" if M <= 2 else "gemv_q4_f32" if M <= 16 else "gemm_f32_mfma")
