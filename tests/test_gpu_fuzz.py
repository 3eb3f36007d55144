"""Seeded random geometries for every operator, against the oracle.

The hand-picked cases in the other GPU files pin each kernel family's edges;
these draw rows, K (whole blocks, multiples of 8 and arbitrary), widths, block
sizes, bit widths, zero-point kinds, optional inputs and dtypes at random
within each entry point's contract, so that the kernel choice and every tail
path meet shapes nobody picked. The draws are fixed by the seed below, and
each case's id names its geometry. Bars are the same as elsewhere: outputs
within ``oracle.tolerance_ok``, gathers and residuals bit-exact.
"""
import numpy as np
import pytest

from oracle import int8a as Q8
from oracle import moe as QM
from oracle import oracle as O
from oracle import quant as QQ

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

SEED = 20261202


def dev(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).cuda()


def host(t):
    return None if t is None else t.detach().cpu().numpy()


def ops():
    from xrgpu_amd import ops as _ops
    return _ops


def check(got, ref, dtype, what=""):
    ok, err, lim = O.tolerance_ok(got, ref, dtype)
    assert ok, f"{what}: max|d|={err} > {lim}"


def weights(rng, K, N, bits, bs, dtype, zp):
    kb = O.k_blocks(K, bs)
    B = rng.integers(0, 256, size=(N, kb, O.blob_bytes(bs, bits)), dtype=np.uint8)
    S = rng.uniform(0.001, 0.02, (N, kb)).astype(dtype)
    Z = None
    if zp == "packed":
        Z = rng.integers(0, 256, size=(N, O.packed_zp_bytes(kb, bits)), dtype=np.uint8)
    elif zp == "float_int":
        Z = rng.integers(0, 1 << bits, size=(N, kb)).astype(dtype)
    elif zp == "float":
        Z = rng.uniform(0, (1 << bits) - 1, (N, kb)).astype(dtype)
    return B, S, Z


def draw_k(rng, bs, kmax=1024):
    kind = rng.integers(0, 3)
    if kind == 0:
        return int(bs * rng.integers(1, max(2, kmax // bs + 1)))  # whole blocks
    if kind == 1:
        return int(8 * rng.integers(1, kmax // 8 + 1))            # a tail inside the last block
    return int(rng.integers(1, kmax + 1))                           # any K


def ids(cases):
    return ["-".join(str(v) for v in c) for c in cases]


# --------------------------------------------------------------------------- MatMulNBits

def _mm_cases(n=32):
    rng = np.random.default_rng(SEED)
    rows = [1, 2, 3, 4, 5, 8, 13, 16, 17, 33, 64, 100, 127, 128, 129, 200, 257, 300]
    out = []
    for _ in range(n):
        M = int(rng.choice(rows))
        if rng.random() < 0.6:  # inside the fast kernels' envelope: 4-bit fp16, whole 32-code chunks
            bs = int(rng.choice([32, 64, 128]))
            K = int(rng.choice([2048, 4096])) if M <= 16 and rng.random() < 0.4 else int(32 * rng.integers(1, 33))
            out.append((M, K, int(rng.integers(1, 520)), 4, bs, str(rng.choice(["none", "packed", "float_int"])),
                        bool(rng.integers(0, 2)), "f16"))
            continue
        bits = int(rng.choice([4, 4, 2, 8]))
        bs = int(rng.choice([16, 32, 64, 128]))
        zp = str(rng.choice(["none", "packed", "float_int", "float"]))
        dt = "f16" if rng.random() < 0.75 else "f32"
        out.append((M, draw_k(rng, bs), int(rng.integers(1, 520)), bits, bs, zp, bool(rng.integers(0, 2)), dt))
    return out


MM = _mm_cases()


@pytest.mark.parametrize("M,K,N,bits,bs,zp,bias,dt", MM, ids=ids(MM))
def test_matmul_nbits_random(gpu, M, K, N, bits, bs, zp, bias, dt):
    rng = np.random.default_rng([SEED, M, K, N, bits, bs])
    dtype = np.float16 if dt == "f16" else np.float32
    A = rng.standard_normal((M, K)).astype(dtype)
    B, S, Z = weights(rng, K, N, bits, bs, dtype, None if zp == "none" else zp)
    b = (rng.standard_normal(N) * 0.1).astype(dtype) if bias else None
    Y = host(ops().matmul_nbits(dev(A), dev(B), dev(S), dev(Z), dev(b), K=K, N=N, bits=bits, block_size=bs))
    check(Y, O.matmul_nbits(A, B, S, Z, b, K=K, N=N, bits=bits, block_size=bs), dtype)


# --------------------------------------------------------------------------- MatMulNBitsQkv / Mlp

def _qkv_cases(n=16):
    rng = np.random.default_rng(SEED + 1)
    out = []
    for _ in range(n):
        bs = int(rng.choice([16, 32, 64, 128]))
        K = int(rng.choice([2048, 4096])) if rng.random() < 0.5 else draw_k(rng, bs)
        out.append((int(rng.integers(1, 17)), K, int(rng.integers(1, 400)), int(rng.integers(1, 200)), bs,
                    str(rng.choice(["none", "packed", "float_int", "float"])), bool(rng.integers(0, 2))))
    return out


QKV = _qkv_cases()


@pytest.mark.parametrize("M,K,Nq,Nkv,bs,zp,skip", QKV, ids=ids(QKV))
def test_qkv_random(gpu, M, K, Nq, Nkv, bs, zp, skip, dt=np.float16):
    rng = np.random.default_rng([SEED, 1, M, K, Nq, Nkv, bs])
    A = rng.standard_normal((M, K)).astype(dt)
    sk = rng.standard_normal((M, K)).astype(dt) if skip else None
    g = rng.uniform(0.5, 1.5, K).astype(dt)
    z = None if zp == "none" else zp
    parts = [weights(rng, K, n, 4, bs, dt, z) for n in (Nq, Nkv, Nkv)]
    Q, Kk, V, R = ops().matmul_nbits_qkv(dev(A), *[dev(x) for p in parts for x in p[:2]], norm_scale=dev(g),
                                         skip=dev(sk), block_size=bs, q_zero_points=dev(parts[0][2]),
                                         k_zero_points=dev(parts[1][2]), v_zero_points=dev(parts[2][2]))
    ref = O.matmul_nbits_qkv(A, parts[0][0], parts[0][1], parts[1][0], parts[1][1], parts[2][0], parts[2][1], K=K,
                             Nq=Nq, Nkv=Nkv, norm_scale=g, skip=sk, block_size=bs, q_zero_points=parts[0][2],
                             k_zero_points=parts[1][2], v_zero_points=parts[2][2])
    for got, exp, nm in zip((Q, Kk, V), ref[:3], "qkv"):
        check(host(got), exp, dt, nm)
    assert np.array_equal(host(R), ref[3])


def _mlp_cases(n=14):
    rng = np.random.default_rng(SEED + 2)
    out = []
    for _ in range(n):
        bs = int(rng.choice([16, 32, 64, 128]))
        out.append((int(rng.integers(1, 17)), draw_k(rng, bs), int(rng.integers(1, 400)), bs, bool(rng.integers(0, 2)),
                    bool(rng.integers(0, 2)), bool(rng.integers(0, 2)), str(rng.choice(["silu", "gelu", "relu"])),
                    bool(rng.integers(0, 2))))
    return out


MLP = _mlp_cases()


@pytest.mark.parametrize("M,K,N,bs,skip,norm,biases,act,res", MLP, ids=ids(MLP))
def test_mlp_random(gpu, M, K, N, bs, skip, norm, biases, act, res, dt=np.float16):
    rng = np.random.default_rng([SEED, 2, M, K, N, bs])
    A = rng.standard_normal((M, K)).astype(dt)
    sk = rng.standard_normal((M, K)).astype(dt) if skip else None
    g = rng.uniform(0.5, 1.5, K).astype(dt) if norm else None
    gB, gS, _ = weights(rng, K, N, 4, bs, dt, None)
    uB, uS, _ = weights(rng, K, N, 4, bs, dt, None)
    gb = (rng.standard_normal(N) * 0.1).astype(dt) if biases else None
    ub = (rng.standard_normal(N) * 0.1).astype(dt) if biases else None
    Y, R = ops().matmul_nbits_mlp(dev(A), dev(gB), dev(gS), dev(uB), dev(uS), skip=dev(sk), norm_scale=dev(g),
                                  gate_bias=dev(gb), up_bias=dev(ub), block_size=bs, activation=act,
                                  want_residual=res)
    ref, r = O.matmul_nbits_mlp(A, gB, gS, uB, uS, K=K, N=N, skip=sk, norm_scale=g, gate_bias=gb, up_bias=ub,
                                block_size=bs, activation=act)
    check(host(Y), ref, dt)
    if res:
        assert np.array_equal(host(R), r)


def _qkv_prefill_cases(n=10):
    """More than 16 rows: the split-K GEMV's row chunks (up to 64 rows, columns
    of 64 or 128 chunks) and the fused GEMM."""
    rng = np.random.default_rng(SEED + 11)
    out = []
    for _ in range(n):
        bs = int(rng.choice([16, 32, 64, 128]))
        K = int(rng.choice([2048, 4096])) if rng.random() < 0.5 else int(bs * rng.integers(1, max(2, 1024 // bs + 1)))
        out.append((int(rng.choice([17, 24, 33, 48, 64, 65, 100, 130, 200])), K, int(rng.integers(1, 300)),
                    int(rng.integers(1, 150)), bs, str(rng.choice(["none", "packed", "float_int"])),
                    bool(rng.integers(0, 2))))
    return out


QKV2 = _qkv_prefill_cases()


@pytest.mark.parametrize("M,K,Nq,Nkv,bs,zp,skip", QKV2, ids=ids(QKV2))
def test_qkv_prefill_random(gpu, M, K, Nq, Nkv, bs, zp, skip):
    test_qkv_random(gpu, M, K, Nq, Nkv, bs, zp, skip)


def _mlp_prefill_cases(n=10):
    rng = np.random.default_rng(SEED + 12)
    out = []
    for _ in range(n):
        bs = int(rng.choice([16, 32, 64, 128]))
        K = int(rng.choice([2048, 4096])) if rng.random() < 0.5 else int(bs * rng.integers(1, max(2, 1024 // bs + 1)))
        out.append((int(rng.choice([17, 24, 33, 48, 64, 65, 100, 130, 200])), K, int(rng.integers(1, 300)), bs,
                    bool(rng.integers(0, 2)), bool(rng.integers(0, 2)), bool(rng.integers(0, 2)),
                    str(rng.choice(["silu", "gelu", "relu", "tanh"])), bool(rng.integers(0, 2))))
    return out


MLP2 = _mlp_prefill_cases()


@pytest.mark.parametrize("M,K,N,bs,skip,norm,biases,act,res", MLP2, ids=ids(MLP2))
def test_mlp_prefill_random(gpu, M, K, N, bs, skip, norm, biases, act, res):
    test_mlp_random(gpu, M, K, N, bs, skip, norm, biases, act, res)


def _f32_fused_rows(rng):
    """Up to four rows (the prologue inside the float32 GEMV), up to 16 (a
    prologue launch, then one GEMV grid), more (one MFMA GEMM grid for every
    projection)."""
    return int(rng.choice([1, 3, 4, 5, 9, 16, 17, 33, 64, 100, 130]))


def _f32_qkv_cases(n=10):
    """Float32 Qkv: K tails and whole blocks, every zero-point kind."""
    rng = np.random.default_rng(SEED + 17)
    out = []
    for _ in range(n):
        bs = int(rng.choice([16, 32, 64, 128]))
        K = int(rng.choice([2048, 4096])) if rng.random() < 0.4 else int(bs * rng.integers(1, max(2, 1024 // bs + 1)))
        out.append((_f32_fused_rows(rng), K, int(rng.integers(1, 400)), int(rng.integers(1, 200)), bs,
                    str(rng.choice(["none", "packed", "float_int", "float"])), bool(rng.integers(0, 2))))
    return out


# plus more than 16 rows with each zero-point kind on the one-grid MFMA GEMM
F32QKV = _f32_qkv_cases() + [(65, 2048, 256, 64, 32, "packed", True), (200, 1024, 300, 100, 64, "float", True),
                             (48, 4096, 128, 128, 128, "float_int", False)]


@pytest.mark.parametrize("M,K,Nq,Nkv,bs,zp,skip", F32QKV, ids=ids(F32QKV))
def test_f32_qkv_random(gpu, M, K, Nq, Nkv, bs, zp, skip):
    test_qkv_random(gpu, M, K, Nq, Nkv, bs, zp, skip, dt=np.float32)


def _f32_mlp_cases(n=10):
    rng = np.random.default_rng(SEED + 18)
    out = []
    for _ in range(n):
        bs = int(rng.choice([16, 32, 64, 128]))
        K = int(rng.choice([2048, 4096])) if rng.random() < 0.4 else int(bs * rng.integers(1, max(2, 1024 // bs + 1)))
        out.append((_f32_fused_rows(rng), K, int(rng.integers(1, 600)), bs, bool(rng.integers(0, 2)),
                    bool(rng.integers(0, 2)), bool(rng.integers(0, 2)), str(rng.choice(["silu", "gelu", "relu", "tanh"])),
                    bool(rng.integers(0, 2))))
    return out


F32MLP = _f32_mlp_cases()


@pytest.mark.parametrize("M,K,N,bs,skip,norm,biases,act,res", F32MLP, ids=ids(F32MLP))
def test_f32_mlp_random(gpu, M, K, N, bs, skip, norm, biases, act, res):
    test_mlp_random(gpu, M, K, N, bs, skip, norm, biases, act, res, dt=np.float32)


def _f32_cases(n=10):
    """Float32 activations, 4-bit, up to four rows: the float32 GEMV (K tails,
    every zero-point kind)."""
    rng = np.random.default_rng(SEED + 13)
    out = []
    for _ in range(n):
        bs = int(rng.choice([16, 32, 64, 128]))
        out.append((int(rng.integers(1, 5)), int(8 * rng.integers(1, 1025)), int(rng.integers(1, 600)), 4, bs,
                    str(rng.choice(["none", "packed", "float_int", "float"])), bool(rng.integers(0, 2)), "f32"))
    return out


MMF32 = _f32_cases()


def _wide_prefill_cases(n, seed, dt, bit_choices):
    """More than 16 rows on the float32-arithmetic MFMA GEMM: blocks of
    32..256 with partial last blocks, no or packed zero points (float zero
    points fall back to the float32 GEMV)."""
    rng = np.random.default_rng(seed)
    q = 4 if dt == "f32" else 8  # K % 4 (float32) or K % 8 (float16)
    out = []
    for _ in range(n):
        bits = int(rng.choice(bit_choices))
        bs = int(rng.choice([32, 64, 128, 256]))
        step = max(64, bs)
        Kd = step * int(rng.integers(1, max(2, 2048 // step + 1)))
        K = Kd - q * int(rng.integers(0, bs // q))  # a partial last block
        out.append((int(rng.choice([17, 33, 64, 65, 100, 130, 200, 300])), K, int(rng.integers(1, 600)), bits, bs,
                    str(rng.choice(["none", "packed", "packed", "float"])), bool(rng.integers(0, 2)), dt))
    return out


# float32 activations with 2-, 4- and 8-bit codes; float16 with 2 and 8
MMF32P = _wide_prefill_cases(12, SEED + 15, "f32", [2, 4, 8]) + _wide_prefill_cases(8, SEED + 16, "f16", [2, 8])


@pytest.mark.parametrize("M,K,N,bits,bs,zp,bias,dt", MMF32P, ids=ids(MMF32P))
def test_matmul_nbits_wide_prefill_random(gpu, M, K, N, bits, bs, zp, bias, dt):
    test_matmul_nbits_random(gpu, M, K, N, bits, bs, zp, bias, dt)


@pytest.mark.parametrize("M,K,N,bits,bs,zp,bias,dt", MMF32, ids=ids(MMF32))
def test_matmul_nbits_f32_random(gpu, M, K, N, bits, bs, zp, bias, dt):
    test_matmul_nbits_random(gpu, M, K, N, bits, bs, zp, bias, dt)


def _prepacked_cases(n=10):
    """Prepacked weights: the prefill GEMM at any row count, K of whole 32-code
    chunks (tails inside a block), every zero-point kind."""
    rng = np.random.default_rng(SEED + 14)
    out = []
    for _ in range(n):
        bs = int(rng.choice([16, 32, 64, 128]))
        while True:
            K = int(8 * rng.integers(1, 129))
            if (-(-K // bs) * bs) % 32 == 0:
                break
        out.append((int(rng.choice([1, 7, 64, 128, 129, 300, 513])), K, int(rng.integers(1, 600)), bs,
                    str(rng.choice(["none", "packed", "float_int", "float"])), bool(rng.integers(0, 2))))
    return out


PKC = _prepacked_cases()


@pytest.mark.parametrize("M,K,N,bs,zp,bias", PKC, ids=ids(PKC))
def test_prepacked_random(gpu, M, K, N, bs, zp, bias):
    rng = np.random.default_rng([SEED, 14, M, K, N, bs])
    A = rng.standard_normal((M, K)).astype(np.float16)
    B, S, Z = weights(rng, K, N, 4, bs, np.float16, None if zp == "none" else zp)
    b = (rng.standard_normal(N) * 0.1).astype(np.float16) if bias else None
    o = ops()
    packed = o.prepack_weights(dev(B), K=K, block_size=bs)
    Y = host(o.matmul_nbits_prepacked(dev(A), packed, dev(S), dev(Z), dev(b), K=K, N=N, block_size=bs))
    check(Y, O.matmul_nbits(A, B, S, Z, b, K=K, N=N, block_size=bs), np.float16)


# --------------------------------------------------------------------------- GatherBlockQuantized / MatMulBnb4

def _gbq_cases(n=16):
    rng = np.random.default_rng(SEED + 3)
    out = []
    for _ in range(n):
        bits = int(rng.choice([4, 8]))
        width = int(rng.integers(1, 600)) * (8 // bits) if rng.random() < 0.5 else int(rng.integers(1, 300)) * 32
        out.append((int(rng.integers(1, 600)), width, bits, int(rng.choice([16, 32, 64, 128])), bool(rng.integers(0, 2)),
                    bool(rng.integers(0, 2)), int(rng.integers(1, 300))))
    return out


GBQ = _gbq_cases()


@pytest.mark.parametrize("rows,width,bits,bs,zp,i64,n", GBQ, ids=ids(GBQ))
def test_gather_block_quantized_random(gpu, rows, width, bits, bs, zp, i64, n):
    rng = np.random.default_rng([SEED, 3, rows, width, bits, bs, n])
    data = rng.integers(0, 256, (rows, width * bits // 8), dtype=np.uint8)
    blocks = (width + bs - 1) // bs
    scales = rng.uniform(-0.5, 0.5, (rows, blocks)).astype(np.float32)
    zps = rng.integers(0, 256, (rows, (blocks * bits + 7) // 8), dtype=np.uint8) if zp else None
    idx = rng.integers(0, rows, n).astype(np.int64 if i64 else np.int32)
    got = host(ops().gather_block_quantized(dev(data), dev(idx), dev(scales), dev(zps), bits=bits, block_size=bs))
    assert np.array_equal(got, QQ.gather_block_quantized(data, idx, scales, zps, bits=bits, block_size=bs))


def _bnb_cases(n=16):
    rng = np.random.default_rng(SEED + 4)
    out = []
    for _ in range(n):
        K = int(32 * rng.integers(1, 65)) if rng.random() < 0.7 else int(rng.integers(1, 600))
        out.append((int(rng.integers(1, 20)), K, int(rng.integers(1, 600)), int(rng.choice([16, 32, 48, 64, 128, 256])),
                    int(rng.integers(0, 2)), str(rng.choice(["f16", "f32"])), int(rng.random() < 0.85)))
    return out


BNB = _bnb_cases()


@pytest.mark.parametrize("M,K,N,bs,qt,dt,tb", BNB, ids=ids(BNB))
def test_matmul_bnb4_random(gpu, M, K, N, bs, qt, dt, tb):
    rng = np.random.default_rng([SEED, 4, M, K, N, bs])
    dtype = np.float16 if dt == "f16" else np.float32
    a = rng.standard_normal((M, K)).astype(dtype)
    b = rng.integers(0, 256, (N * K + 1) // 2, dtype=np.uint8)
    absmax = rng.uniform(0.05, 1.5, (N * K + bs - 1) // bs).astype(dtype)
    got = host(ops().matmul_bnb4(dev(a), dev(b), dev(absmax), K=K, N=N, block_size=bs, quant_type=qt, trans_b=tb))
    check(got, QQ.matmul_bnb4(a, b, absmax, K=K, N=N, block_size=bs, quant_type=qt, trans_b=tb), dtype)


# --------------------------------------------------------------------------- QMoE

def _moe_cases(n=12):
    rng = np.random.default_rng(SEED + 5)
    out = []
    for _ in range(n):
        bits = int(rng.choice([4, 8]))
        bs = int(rng.choice([0, 16, 32, 64]))
        if bs == 0 and rng.random() < 0.35:  # rows that are not whole 16-byte chunks: the scalar kernels
            H, I = int(8 * (2 * rng.integers(1, 40) + 1)), int(8 * (2 * rng.integers(1, 60) + 1))
        else:
            unit = max(bs, 32)
            H = int(unit * rng.integers(1, max(2, 1024 // unit)))
            I = int(unit * rng.integers(1, max(2, 1536 // unit)))
        E = int(rng.integers(1, 9))
        act = str(rng.choice(["swiglu", "relu"]))
        limit = float(rng.choice([0.0, 2.0])) if act == "swiglu" else 0.0
        out.append((int(rng.integers(1, 7)), H, I, E, int(rng.integers(1, E + 1)), bits, bs, act, limit))
    return out


MOE = _moe_cases()


@pytest.mark.parametrize("T,H,I,E,k,bits,bs,act,limit", MOE, ids=ids(MOE))
def test_qmoe_random(gpu, T, H, I, E, k, bits, bs, act, limit):
    rng = np.random.default_rng([SEED, 5, T, H, I, E, k, bits, bs])
    sw = act == "swiglu"
    F1 = 2 * I if sw else I
    i = {"inputT": (rng.standard_normal((T, H)) * 0.5).astype(np.float32),
         "routerT": rng.standard_normal((T, E)).astype(np.float32),
         "fc1T": rng.integers(0, 256, (E, F1, H * bits // 8), dtype=np.uint8),
         "fc2T": rng.integers(0, 256, (E, H, I * bits // 8), dtype=np.uint8),
         "fc1ScalesT": rng.uniform(0.01, 0.05, (E, F1, H // bs) if bs else (E, F1)).astype(np.float32),
         "fc2ScalesT": rng.uniform(0.01, 0.05, (E, H, I // bs) if bs else (E, H)).astype(np.float32)}
    at = dict(k=k, activation=act, swiglu_fusion=1 if sw else 0, bits=bits, block_size=bs,
              alpha=1.702 if sw else 1.0, beta=1.0 if sw else 0.0, swiglu_limit=limit if limit else None)
    got = host(ops().qmoe(dev(i["inputT"]), dev(i["routerT"]), dev(i["fc1T"]), dev(i["fc1ScalesT"]), dev(i["fc2T"]),
                          dev(i["fc2ScalesT"]), k=k, activation=act, swiglu_fusion=at["swiglu_fusion"],
                          expert_weight_bits=bits, block_size=bs, activation_alpha=at["alpha"],
                          activation_beta=at["beta"], swiglu_limit=at["swiglu_limit"]))
    ref = QM.qmoe(i["inputT"], i["routerT"], i["fc1T"], i["fc1ScalesT"], i["fc2T"], i["fc2ScalesT"], **at)
    check(got, ref, np.float32)


# --------------------------------------------------------------------------- opt-in int8 activations

def _i8_cases(n=12):
    rng = np.random.default_rng(SEED + 6)
    out = []
    for _ in range(n):
        bs = int(rng.choice([32, 64, 128]))
        out.append((int(rng.integers(1, 9)), int(128 * rng.integers(1, 17)), int(rng.integers(1, 300)), bs,
                    bool(rng.integers(0, 2)), bool(rng.integers(0, 2)), str(rng.choice(["f16", "f32"]))))
    return out


I8 = _i8_cases()


@pytest.mark.parametrize("M,K,N,bs,zp,bias,dt", I8, ids=ids(I8))
def test_int8a_random(gpu, M, K, N, bs, zp, bias, dt):
    rng = np.random.default_rng([SEED, 6, M, K, N, bs])
    dtype = np.float16 if dt == "f16" else np.float32
    A = rng.standard_normal((M, K)).astype(dtype)
    B, S, Z = weights(rng, K, N, 4, bs, dtype, "packed" if zp else None)
    b = (rng.standard_normal(N) * 0.1).astype(dtype) if bias else None
    got = host(ops().matmul_nbits_int8a(dev(A), dev(B), dev(S), dev(Z), dev(b), K=K, N=N, block_size=bs))
    check(got, Q8.matmul_nbits_int8a(A, B, S, Z, b, K=K, N=N, block_size=bs), dtype)
