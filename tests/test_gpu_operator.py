"""GPU: the request-level lifecycle (prepare / run / read_outputs / info /
close) against the oracle, and its failure behaviour (closed and poisoned
operators, readback before run, a host-forced time-out)."""
import numpy as np
import pytest

from oracle import oracle as O
from xrgpu_amd import operator as op

pytestmark = pytest.mark.gpu

MNB, QKV, MLP = "com.microsoft.MatMulNBits", "com.microsoft.MatMulNBitsQkv", "com.microsoft.MatMulNBitsMlp"


def rand_mnb(rng, M, K, N, bs, zp=True, bias=True, dtype=np.float16):
    kb = K // bs
    ins = dict(aT=rng.standard_normal((M, K)).astype(dtype),
               bT=rng.integers(0, 256, (N, kb, bs // 2), dtype=np.uint8),
               scalesT=rng.uniform(0.001, 0.02, (N, kb)).astype(dtype))
    if zp:
        ins["zeroPointsT"] = rng.integers(0, 256, (N, (kb + 1) // 2), dtype=np.uint8)
    if bias:
        ins["biasT"] = (rng.standard_normal(N) * 0.1).astype(dtype)
    return ins


def request(opname, ins, attrs, requested=()):
    return op.Request(opname, [op.Tensor(k, v) for k, v in ins.items()], attrs=attrs,
                      requested_outputs=list(requested))


@pytest.mark.parametrize("M,K,N,bs", [(1, 4096, 512, 32), (64, 1024, 256, 128), (3, 96, 40, 32)])
def test_matmul_lifecycle_matches_oracle(gpu, M, K, N, bs):
    rng = np.random.default_rng(M + K + N)
    ins = rand_mnb(rng, M, K, N, bs)
    with op.Operator.prepare("", request(MNB, ins, {"N": N, "block_size": bs}), op.Options(profiling=True)) as o:
        o.run()
        o.run()  # the prepared inputs are reused
        (y,) = o.read_outputs()
        info = o.info()
    ref = O.matmul_nbits(ins["aT"], ins["bT"], ins["scalesT"], ins["zeroPointsT"], ins["biasT"], K=K, N=N,
                         block_size=bs)
    assert y.name == "yT" and y.data.shape == (M, N) and y.data.dtype == np.float16
    ok, err, lim = O.tolerance_ok(y.data, ref, np.float16)
    assert ok, (err, lim)
    assert info["backend"] == "hip" and info["operation"] == MNB and info["executed"] and not info["closed"]
    assert info["cpu_compute_fallback"] is False and info["dispatch_count"] == 1
    assert info["execution_ms"] > 0 and info["gpu_ms"] is not None and info["gpu_ms"] > 0
    assert "gfx950" in info["device"]


def test_prefill_lifecycle_prepacks_the_weights(gpu):
    """A request that reaches the 256 x 256 GEMM (512 rows, 128 tiles) gets
    its weights prepacked at prepare; the result meets the oracle, and a
    memory limit that leaves no room for the packed copy runs the unpacked
    GEMM with the same tolerance."""
    rng = np.random.default_rng(77)
    M, K, N, bs = 512, 128, 16384, 64
    ins = rand_mnb(rng, M, K, N, bs)
    ref = O.matmul_nbits(ins["aT"], ins["bT"], ins["scalesT"], ins["zeroPointsT"], ins["biasT"], K=K, N=N,
                         block_size=bs)
    arena = sum(v.nbytes for v in ins.values()) + M * N * 2
    for limit, kernel in ((256 << 20, "gemm_q4_big_prepacked"), (arena + (64 << 10), "gemm_q4_big")):
        with op.Operator.prepare("", request(MNB, ins, {"N": N, "block_size": bs}),
                                 op.Options(memory_limit_bytes=limit)) as o:
            o.run()
            (y,) = o.read_outputs()
            assert o.info()["kernel"] == kernel
        ok, err, lim = O.tolerance_ok(y.data, ref, np.float16)
        assert ok, (kernel, err, lim)


def test_splitk_lifecycle_runs_twice_on_its_workspace(gpu):
    """A request with few output tiles (40 rows, N = 512: 4 tiles) runs the
    split-K GEMM on a workspace in the operator's arena; the second run finds
    the counters zeroed by the first and gives the same bits."""
    from xrgpu_amd import _native as nat
    rng = np.random.default_rng(31)
    M, K, N, bs = 40, 8192, 512, 64
    assert nat.lib().xrmm_matmul_nbits_workspace_bytes(M, K, N, 4, bs, nat.F16) > 0
    ins = rand_mnb(rng, M, K, N, bs)
    with op.Operator.prepare("", request(MNB, ins, {"N": N, "block_size": bs})) as o:
        o.run()
        (y1,) = o.read_outputs()
        o.run()
        (y2,) = o.read_outputs()
    ref = O.matmul_nbits(ins["aT"], ins["bT"], ins["scalesT"], ins["zeroPointsT"], ins["biasT"], K=K, N=N,
                         block_size=bs)
    ok, err, lim = O.tolerance_ok(y1.data, ref, np.float16)
    assert ok, (err, lim)
    assert np.array_equal(y1.data.view(np.uint16), y2.data.view(np.uint16))


def test_splitk_workspace_is_optional_under_the_memory_limit(gpu):
    """A memory limit just above the request's own bytes leaves no room for
    the split-K workspace: prepare still succeeds and the run (unsplit)
    meets the oracle."""
    from xrgpu_amd import _native as nat
    rng = np.random.default_rng(32)
    M, K, N, bs = 40, 8192, 512, 64
    ws = nat.lib().xrmm_matmul_nbits_workspace_bytes(M, K, N, 4, bs, nat.F16)
    assert ws > 4096
    ins = rand_mnb(rng, M, K, N, bs)
    data = sum((v.nbytes + 255) // 256 * 256 for v in ins.values()) + (M * N * 2 + 255) // 256 * 256
    with op.Operator.prepare("", request(MNB, ins, {"N": N, "block_size": bs}),
                             op.Options(memory_limit_bytes=data + 1024)) as o:
        o.run()
        (y,) = o.read_outputs()
    ref = O.matmul_nbits(ins["aT"], ins["bT"], ins["scalesT"], ins["zeroPointsT"], ins["biasT"], K=K, N=N,
                         block_size=bs)
    ok, err, lim = O.tolerance_ok(y.data, ref, np.float16)
    assert ok, (err, lim)
    with pytest.raises(op.XrmmInvalid, match="Extended heap memory limit exceeded"):
        op.Operator.prepare("", request(MNB, ins, {"N": N, "block_size": bs}),
                            op.Options(memory_limit_bytes=data - 256))


def test_requested_float32_storage_holds_the_float16_values(gpu):
    rng = np.random.default_rng(1)
    ins = rand_mnb(rng, 2, 256, 64, 32)
    want = [op.Tensor("yT", shape=(2, 64), dtype="float16", storage_dtype="float32")]
    with op.Operator.prepare("", request(MNB, ins, {"N": 64}, want)) as o:
        o.run()
        (y32,) = o.read_outputs()
    with op.Operator.prepare("", request(MNB, ins, {"N": 64})) as o:
        o.run()
        (y16,) = o.read_outputs()
    assert y32.data.dtype == np.float32 and np.array_equal(y32.data, y16.data.astype(np.float32))


def test_float32_input_storage_of_float16_logical_tensor(gpu):
    """A float16 logical tensor supplied as float32 storage is rounded once
    (RNE) on upload, like the reference's logical_bits (planner.cpp:27)."""
    rng = np.random.default_rng(2)
    ins = rand_mnb(rng, 1, 128, 16, 32, zp=False, bias=False)
    a32 = rng.standard_normal((1, 128)).astype(np.float32)
    ins16 = dict(ins, aT=a32.astype(np.float16))
    tensors = [op.Tensor("aT", a32, dtype="float16", storage_dtype="float32"),
               op.Tensor("bT", ins["bT"]), op.Tensor("scalesT", ins["scalesT"])]
    with op.Operator.prepare("", op.Request(MNB, tensors, attrs={"N": 16})) as o:
        o.run()
        (y,) = o.read_outputs()
    with op.Operator.prepare("", request(MNB, ins16, {"N": 16})) as o:
        o.run()
        (y16,) = o.read_outputs()
    assert np.array_equal(y.data, y16.data)


def test_qkv_lifecycle_with_residual(gpu):
    rng = np.random.default_rng(3)
    M, K, Nq, Nkv, bs = 4, 512, 128, 64, 64
    kb = K // bs
    ins = dict(aT=rng.standard_normal((M, K)).astype(np.float16), skipT=rng.standard_normal((M, K)).astype(np.float16),
               normScaleT=rng.uniform(0.5, 1.5, K).astype(np.float16))
    for p, n in (("q", Nq), ("k", Nkv), ("v", Nkv)):
        ins[p + "BT"] = rng.integers(0, 256, (n, kb, bs // 2), dtype=np.uint8)
        ins[p + "ScalesT"] = rng.uniform(0.001, 0.02, (n, kb)).astype(np.float16)
    want = [op.Tensor(n, shape=s, dtype="float16") for n, s in
            (("qT", (M, Nq)), ("kT", (M, Nkv)), ("vT", (M, Nkv)), ("residualT", (M, K)))]
    with op.Operator.prepare("", request(QKV, ins, {"Nq": Nq, "Nkv": Nkv, "block_size": bs}, want)) as o:
        o.run()
        outs = o.read_outputs()
    ref = O.matmul_nbits_qkv(ins["aT"], ins["qBT"], ins["qScalesT"], ins["kBT"], ins["kScalesT"], ins["vBT"],
                             ins["vScalesT"], K=K, Nq=Nq, Nkv=Nkv, norm_scale=ins["normScaleT"], skip=ins["skipT"],
                             block_size=bs)
    assert [t.name for t in outs] == ["qT", "kT", "vT", "residualT"]
    for t, r in zip(outs[:3], ref[:3]):
        assert O.tolerance_ok(t.data, r, np.float16)[0], t.name
    assert np.array_equal(outs[3].data, ref[3])


def test_mlp_lifecycle(gpu):
    rng = np.random.default_rng(4)
    M, K, N, bs = 16, 512, 96, 32
    kb = K // bs
    ins = dict(aT=rng.standard_normal((M, K)).astype(np.float16))
    for p in ("gate", "up"):
        ins[p + "BT"] = rng.integers(0, 256, (N, kb, bs // 2), dtype=np.uint8)
        ins[p + "ScalesT"] = rng.uniform(0.001, 0.02, (N, kb)).astype(np.float16)
    with op.Operator.prepare("", request(MLP, ins, {"N": N, "block_size": bs, "activation": "silu"})) as o:
        o.run()
        (y,) = o.read_outputs()
    ref, _ = O.matmul_nbits_mlp(ins["aT"], ins["gateBT"], ins["gateScalesT"], ins["upBT"], ins["upScalesT"], K=K, N=N,
                                block_size=bs)
    assert O.tolerance_ok(y.data, ref, np.float16)[0]


def test_failure_states(gpu):
    rng = np.random.default_rng(5)
    ins = rand_mnb(rng, 1, 256, 32, 32)
    o = op.Operator.prepare("", request(MNB, ins, {"N": 32}))
    with pytest.raises(op.XrmmError, match="Run extended operator before readback"):
        o.read_outputs()
    o.run()
    o.close()
    assert o.info()["closed"] is True
    with pytest.raises(op.XrmmError, match="closed"):
        o.run()
    with pytest.raises(op.XrmmError, match="closed"):
        o.read_outputs()


def test_host_forced_timeout_poisons_until_close(gpu):
    """A 1 ns limit expires while a ~50 us launch is still running; the
    kernel itself completes normally and close() waits for it."""
    rng = np.random.default_rng(6)
    ins = rand_mnb(rng, 512, 4096, 4096, 128)
    o = op.Operator.prepare("", request(MNB, ins, {"N": 4096, "block_size": 128}), op.Options(timeout_ns=1))
    with pytest.raises(op.XrmmError, match="timed out"):
        o.run()
    with pytest.raises(op.XrmmError, match="failed and must be closed"):
        o.run()
    o.close()
    assert o.info()["closed"] is True


BNB, QMOE, GBQ = "com.microsoft.MatMulBnb4", "com.microsoft.QMoE", "com.microsoft.GatherBlockQuantized"


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_bnb4_lifecycle(gpu, dtype):
    from oracle import quant as Q
    rng = np.random.default_rng(5)
    M, K, N, bs = 2, 512, 96, 64
    ins = dict(aT=rng.standard_normal((M, K)).astype(dtype), bT=rng.integers(0, 256, N * K // 2, dtype=np.uint8),
               absmaxT=rng.uniform(0.1, 1.0, N * K // bs).astype(dtype))
    with op.Operator.prepare("", request(BNB, ins, {"K": K, "N": N, "block_size": bs, "quant_type": 0})) as o:
        o.run()
        (y,) = o.read_outputs()
        assert o.info()["kernel"] == "bnb4_gemv"
    ref = Q.matmul_bnb4(ins["aT"], ins["bT"], ins["absmaxT"], K=K, N=N, block_size=bs, quant_type=0)
    ok, err, lim = O.tolerance_ok(y.data, ref, dtype)
    assert ok, (err, lim)


def test_qmoe_lifecycle(gpu):
    from oracle import moe as QM
    rng = np.random.default_rng(6)
    T_, H, I, E = 3, 256, 128, 4
    ins = dict(inputT=rng.standard_normal((1, T_, H)).astype(np.float32),
               routerT=rng.standard_normal((T_, E)).astype(np.float32),
               fc1T=rng.integers(0, 256, (E, 2 * I, H // 2), dtype=np.uint8),
               fc1ScalesT=rng.uniform(0.01, 0.05, (E, 2 * I, H // 32)).astype(np.float32),
               fc2T=rng.integers(0, 256, (E, H, I // 2), dtype=np.uint8),
               fc2ScalesT=rng.uniform(0.01, 0.05, (E, H, I // 32)).astype(np.float32))
    attrs = {"k": 2, "activation_type": "swiglu", "swiglu_fusion": 1, "block_size": 32, "activation_alpha": 1.702,
             "activation_beta": 1.0, "swiglu_limit": 7.0}
    with op.Operator.prepare("", request(QMOE, ins, attrs)) as o:
        o.run()
        o.run()
        (y,) = o.read_outputs()
        info = o.info()
    assert info["kernel"] == "qmoe_rows" and info["dispatch_count"] == 1
    ref = QM.qmoe(ins["inputT"], ins["routerT"], ins["fc1T"], ins["fc1ScalesT"], ins["fc2T"], ins["fc2ScalesT"], k=2,
                  activation="swiglu", swiglu_fusion=1, bits=4, block_size=32, alpha=1.702, beta=1.0, swiglu_limit=7.0)
    assert y.data.shape == (1, T_, H)
    ok, err, lim = O.tolerance_ok(y.data, ref, np.float32)
    assert ok, (err, lim)


def test_gbq_lifecycle_and_index_failure(gpu):
    from oracle import quant as Q
    rng = np.random.default_rng(8)
    rows, pcols, bs = 40, 64, 32
    data = rng.integers(0, 256, (rows, pcols), dtype=np.uint8)
    scales = rng.uniform(-1, 1, (rows, pcols * 2 // bs)).astype(np.float32)
    zps = rng.integers(0, 256, (rows, pcols * 2 // bs // 2), dtype=np.uint8)
    idx = np.array([3, 39, 0, 3], np.int64)
    ins = dict(dataT=data, indicesT=idx, scalesT=scales, zeroPointsT=zps)
    with op.Operator.prepare("", request(GBQ, ins, {"bits": 4, "block_size": bs})) as o:
        o.run()
        (y,) = o.read_outputs()
        assert o.info()["kernel"] == "gbq_words"
    assert np.array_equal(y.data, Q.gather_block_quantized(data, idx, scales, zps, bits=4, block_size=bs))
    bad = dict(ins, indicesT=np.array([1, rows], np.int64))
    o = op.Operator.prepare("", request(GBQ, bad, {"bits": 4, "block_size": bs}))
    with pytest.raises(op.XrmmError, match="GPU operator contract validation failed: code 55"):
        o.run()
    with pytest.raises(op.XrmmError, match="failed and must be closed"):
        o.run()
    o.close()
