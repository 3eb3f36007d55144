"""Request-level plan() through the C ABI, without a device: contract checks,
attribute defaults, args-over-attrs precedence, output shapes and requested
outputs (kernels/_shared/extended/planner.cpp:67-93, complex_plan.cpp:117-129,
contract_data.h:659-663,718-751,821-827), for the MatMulNBits family,
MatMulBnb4, QMoE and GatherBlockQuantized (the latter three with the
reference planner's messages)."""
import numpy as np
import pytest

from xrgpu_amd import operator as op

MNB, QKV, MLP = "com.microsoft.MatMulNBits", "com.microsoft.MatMulNBitsQkv", "com.microsoft.MatMulNBitsMlp"


def T(name, shape, dtype="float16"):
    return op.Tensor(name, np.zeros(shape, np.dtype(dtype)))


def mnb(K=64, N=8, bs=32, lead=(2, 3), dtype="float16", extra=()):
    kb = (K + bs - 1) // bs
    return [T("aT", lead + (K,), dtype), T("bT", (N, kb, bs // 2), "uint8"), T("scalesT", (N, kb), dtype), *extra]


def test_output_shape_folds_leading_axes():
    outs = op.plan(op.Request(MNB, mnb(), attrs={"N": 8, "block_size": 32}))
    assert [(t.name, t.shape, t.dtype, t.storage_dtype) for t in outs] == [("yT", (2, 3, 8), "float16", "float16")]


def test_K_defaults_to_last_dim_and_block_size_to_32():
    outs = op.plan(op.Request(MNB, mnb(K=64, bs=32), attrs={"N": 8}))
    assert outs[0].shape == (2, 3, 8)


def test_args_override_attrs():
    req = op.Request(MNB, mnb(N=8), attrs={"N": 5, "block_size": 32}, args={"N": 8})
    assert op.plan(req)[0].shape[-1] == 8
    with pytest.raises(op.XrmmInvalid, match="bT must have shape"):
        op.plan(op.Request(MNB, mnb(N=8), attrs={"N": 8, "block_size": 32}, args={"N": 5}))


def test_float_integer_attribute_accepted_and_fraction_rejected():
    assert op.plan(op.Request(MNB, mnb(), attrs={"N": 8.0}))[0].shape[-1] == 8
    with pytest.raises(op.XrmmInvalid, match="Integer attribute required: N"):
        op.plan(op.Request(MNB, mnb(), attrs={"N": 8.5}))


@pytest.mark.parametrize("mutate,msg", [
    (lambda ins: ins[:1], "Missing required frozen-contract input: bT"),
    (lambda ins: ins + [T("gammaT", (64,))], "Unknown input outside frozen contract: gammaT"),
    (lambda ins: [T("aT", (2, 3, 64), "int32")] + ins[1:], "Logical dtype outside frozen contract: aT"),
    (lambda ins: ins[:2] + [T("scalesT", (8, 2), "float32")], "Type variable differs between tensors: T1"),
    (lambda ins: ins[:1] + [T("bT", (8, 32), "uint8")] + ins[2:], "Rank outside frozen contract: bT"),
    (lambda ins: ins + [T("biasT", (7,))], "biasT must have shape"),
    (lambda ins: ins + [ins[0]], "Duplicate"),
])
def test_contract_violations_are_invalid(mutate, msg):
    with pytest.raises(op.XrmmInvalid, match=msg):
        op.plan(op.Request(MNB, mutate(mnb()), attrs={"N": 8}))


def test_geometry_errors():
    with pytest.raises(op.XrmmInvalid, match="Packed matmul N required"):
        op.plan(op.Request(MNB, mnb(), attrs={}))
    with pytest.raises(op.XrmmInvalid, match="Invalid packed matmul geometry"):
        op.plan(op.Request(MNB, mnb(), attrs={"N": 8, "block_size": 0}))
    with pytest.raises(op.XrmmInvalid, match="bits must be 2, 4 or 8"):
        op.plan(op.Request(MNB, mnb(), attrs={"N": 8, "bits": 3}))
    with pytest.raises(op.XrmmInvalid, match="Unsupported extended operator"):
        op.plan(op.Request("com.microsoft.MatMulNBitsFp8", mnb(), attrs={"N": 8}))


def test_packed_and_float_zero_point_shapes():
    zp_packed = T("zeroPointsT", (8, 1), "uint8")  # kb = 2 blocks, 4-bit: 1 byte per row
    assert op.plan(op.Request(MNB, mnb(extra=(zp_packed,)), attrs={"N": 8}))[0].shape == (2, 3, 8)
    zp_float = T("zeroPointsT", (8, 2), "float32")  # T3 may differ from T1
    assert op.plan(op.Request(MNB, mnb(extra=(zp_float,)), attrs={"N": 8}))[0].shape == (2, 3, 8)
    with pytest.raises(op.XrmmInvalid, match="zeroPointsT must have shape"):
        op.plan(op.Request(MNB, mnb(extra=(T("zeroPointsT", (8, 2), "uint8"),)), attrs={"N": 8}))


def test_requested_outputs_select_storage_and_are_checked():
    want = [op.Tensor("yT", shape=(2, 3, 8), dtype="float16", storage_dtype="float32")]
    outs = op.plan(op.Request(MNB, mnb(), attrs={"N": 8}, requested_outputs=want))
    assert outs[0].storage_dtype == "float32"
    bad = [op.Tensor("yT", shape=(2, 3, 9), dtype="float16")]
    with pytest.raises(op.XrmmInvalid, match="Requested output shape differs from plan"):
        op.plan(op.Request(MNB, mnb(), attrs={"N": 8}, requested_outputs=bad))
    bad = [op.Tensor("yT", shape=(2, 3, 8), dtype="float32")]
    with pytest.raises(op.XrmmInvalid, match="name/type differs"):
        op.plan(op.Request(MNB, mnb(), attrs={"N": 8}, requested_outputs=bad))


def qkv_inputs(K=64, Nq=16, Nkv=8, bs=32):
    kb = K // bs
    ins = [T("aT", (4, K)), T("normScaleT", (K,))]
    for p, n in (("q", Nq), ("k", Nkv), ("v", Nkv)):
        ins += [T(p + "BT", (n, kb, bs // 2), "uint8"), T(p + "ScalesT", (n, kb))]
    return ins


def test_qkv_outputs_and_optional_residual():
    outs = op.plan(op.Request(QKV, qkv_inputs(), attrs={"Nq": 16, "Nkv": 8}))
    assert [(t.name, t.shape) for t in outs] == [("qT", (4, 16)), ("kT", (4, 8)), ("vT", (4, 8))]
    want = [op.Tensor(n, shape=s, dtype="float16") for n, s in
            (("qT", (4, 16)), ("kT", (4, 8)), ("vT", (4, 8)), ("residualT", (4, 64)))]
    outs = op.plan(op.Request(QKV, qkv_inputs(), attrs={"Nq": 16, "Nkv": 8}, requested_outputs=want))
    assert [t.name for t in outs] == ["qT", "kT", "vT", "residualT"]
    with pytest.raises(op.XrmmInvalid, match="Missing required frozen-contract input: normScaleT"):
        op.plan(op.Request(QKV, [t for t in qkv_inputs() if t.name != "normScaleT"], attrs={"Nq": 16, "Nkv": 8}))


def test_mlp_activation_names():
    K, N, bs = 64, 8, 32
    ins = [T("aT", (3, K))] + [T(p + s, sh, dt) for p in ("gate", "up") for s, sh, dt in
                                (("BT", (N, 2, 16), "uint8"), ("ScalesT", (N, 2), "float16"))]
    for act in ("silu", "swish", "gelu", "relu", "tanh", "sigmoid", "identity", "none", "swiglu"):
        assert op.plan(op.Request(MLP, ins, attrs={"N": N, "activation": act}))[0].shape == (3, N)
    with pytest.raises(op.XrmmInvalid, match="Unknown fused activation: mish"):
        op.plan(op.Request(MLP, ins, attrs={"N": N, "activation": "mish"}))


def test_prepare_rejects_byte_count_and_memory_limit_before_touching_a_device():
    req = op.Request(MNB, mnb(), attrs={"N": 8})
    req.inputs[0].data = req.inputs[0].data.reshape(-1)[:-1]  # one element short
    with pytest.raises(op.XrmmInvalid, match="byte count mismatch: aT"):
        op.Operator.prepare("", req)
    with pytest.raises(op.XrmmInvalid, match="memory limit exceeded"):
        op.Operator.prepare("", op.Request(MNB, mnb(), attrs={"N": 8}), op.Options(memory_limit_bytes=64))
    with pytest.raises(op.XrmmInvalid, match="Positive extended runtime limits"):
        op.Operator.prepare("", op.Request(MNB, mnb(), attrs={"N": 8}), op.Options(timeout_ns=0))


BNB, QMOE, GBQ = "com.microsoft.MatMulBnb4", "com.microsoft.QMoE", "com.microsoft.GatherBlockQuantized"


def bnb(M=3, K=64, N=8, bs=32, dtype="float16"):
    return [T("aT", (M, K), dtype), T("bT", ((N * K + 1) // 2,), "uint8"), T("absmaxT", ((N * K + bs - 1) // bs,), dtype)]


def test_bnb4_plan_and_checks():
    outs = op.plan(op.Request(BNB, bnb(), attrs={"K": 64, "N": 8, "block_size": 32}))
    assert [(t.name, t.shape, t.dtype) for t in outs] == [("yT", (3, 8), "float16")]
    with pytest.raises(op.XrmmInvalid, match="Packed matmul N required"):
        op.plan(op.Request(BNB, bnb(), attrs={"K": 64}))
    with pytest.raises(op.XrmmInvalid, match="quant_type"):
        op.plan(op.Request(BNB, bnb(), attrs={"N": 8, "quant_type": 2}))
    with pytest.raises(op.XrmmInvalid, match="Type variable differs between tensors: T1"):
        op.plan(op.Request(BNB, bnb()[:2] + [T("absmaxT", (16,), "float32")], attrs={"N": 8}))
    with pytest.raises(op.XrmmInvalid, match="Rank outside frozen contract: aT"):
        op.plan(op.Request(BNB, [T("aT", (1, 3, 64))] + bnb()[1:], attrs={"N": 8}))
    with pytest.raises(op.XrmmInvalid, match="absmaxT holds fewer"):
        op.plan(op.Request(BNB, bnb(bs=32), attrs={"N": 8, "block_size": 16}))


def qmoe_ins(T_=(2, 3), H=64, I=32, E=4, bits=4, bs=0, swiglu=True):
    F1 = 2 * I if swiglu else I
    sc = lambda rows, cols: T("", (E, rows, cols // bs) if bs else (E, rows), "float32")  # noqa: E731
    s1, s2 = sc(F1, H), sc(H, I)
    s1.name, s2.name = "fc1ScalesT", "fc2ScalesT"
    return [T("inputT", T_ + (H,), "float32"), T("routerT", (int(np.prod(T_)), E), "float32"),
            T("fc1T", (E, F1, H * bits // 8), "uint8"), s1, T("fc2T", (E, H, I * bits // 8), "uint8"), s2]


SW = {"k": 2, "activation_type": "swiglu", "swiglu_fusion": 1}


def test_qmoe_plan_shape_and_reference_messages():
    outs = op.plan(op.Request(QMOE, qmoe_ins(), attrs=SW))
    assert [(t.name, t.shape, t.dtype) for t in outs] == [("outputT", (2, 3, 64), "float32")]
    assert op.plan(op.Request(QMOE, qmoe_ins(bs=16), attrs=dict(SW, block_size=16)))[0].shape == (2, 3, 64)
    cases = [
        (qmoe_ins(), dict(SW, k=5), "Invalid MoE input or routing geometry"),
        (qmoe_ins(), dict(SW, use_sparse_mixer=1), "Invalid MoE input or routing geometry"),
        (qmoe_ins(), {"k": 2, "activation_type": "swiglu"}, "Invalid quantized SwiGLU fusion"),
        (qmoe_ins(swiglu=False), {"k": 1, "swiglu_fusion": 1}, "Invalid quantized SwiGLU fusion"),
        (qmoe_ins(), dict(SW, expert_weight_bits=8), "Invalid packed expert projection"),
        (qmoe_ins(), dict(SW, expert_weight_bits=2), "Unsupported QMoE integer layout"),
        (qmoe_ins(), dict(SW, weights_prepacked=1), "Unsupported QMoE integer layout"),
        (qmoe_ins(bs=16), dict(SW, block_size=24), "Invalid quantized expert block size"),
        (qmoe_ins(bs=16), SW, "Invalid quantized expert scales"),
    ]
    for ins, attrs, msg in cases:
        with pytest.raises(op.XrmmInvalid, match=msg):
            op.plan(op.Request(QMOE, ins, attrs=attrs))
    bad = qmoe_ins()
    bad[4] = T("fc2T", (4, 63, 16), "uint8")
    with pytest.raises(op.XrmmInvalid, match="Invalid MoE weight geometry"):
        op.plan(op.Request(QMOE, bad, attrs=SW))


def gbq_ins(rows=10, pcols=32, n=5, bits=4, bs=16, idx="int64", zp=False):
    width = pcols * 8 // bits
    blocks = (width + bs - 1) // bs
    ins = [T("dataT", (rows, pcols), "uint8"), T("indicesT", (n,), idx), T("scalesT", (rows, blocks), "float32")]
    if zp:
        ins.append(T("zeroPointsT", (rows, (blocks * bits + 7) // 8), "uint8"))
    return ins


def test_gbq_plan_and_checks():
    outs = op.plan(op.Request(GBQ, gbq_ins(), attrs={"bits": 4, "block_size": 16}))
    assert [(t.name, t.shape, t.dtype) for t in outs] == [("outputT", (5, 64), "float32")]
    assert op.plan(op.Request(GBQ, gbq_ins(zp=True), attrs={"bits": 4, "block_size": 16}))[0].shape == (5, 64)
    with pytest.raises(op.XrmmInvalid, match="Logical dtype outside frozen contract: indicesT"):
        op.plan(op.Request(GBQ, gbq_ins(idx="int32"), attrs={"block_size": 16}))  # Tind = int64 (contract_data.h:660)
    assert op.plan(op.Request(GBQ, gbq_ins(bs=128, bits=8), attrs={"bits": 8}))[0].shape == (5, 32)  # defaults
    for attrs in ({"bits": 2, "block_size": 16}, {"block_size": 8}, {"block_size": 48}, {"block_size": 16, "gather_axis": 1},
                  {"block_size": 16, "quantize_axis": 0}):
        with pytest.raises(op.XrmmInvalid, match="Unsupported GatherBlockQuantized geometry"):
            op.plan(op.Request(GBQ, gbq_ins(), attrs=attrs))
    with pytest.raises(op.XrmmInvalid, match="Logical dtype outside frozen contract: indicesT"):
        op.plan(op.Request(GBQ, gbq_ins(idx="int16"), attrs={"block_size": 16}))
    with pytest.raises(op.XrmmInvalid, match="scalesT must have shape"):
        op.plan(op.Request(GBQ, gbq_ins(bs=32), attrs={"block_size": 16}))
